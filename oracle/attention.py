"""Paged attention oracle (numpy, fp64). Test infrastructure only.

Restates ``ascend-kernel/csrc/ops/fa_fp32_stage1/test/fa_fp32_ref.py`` (the
reference's fp64 semantic model of the stage-1 kernel) without ml_dtypes:

* ``gather_kv``      -- fa_fp32_ref.py:68-79: logical token j of a request lives at
                        pool[block_table[b, j // 128], j % 128].
* ``stage1``         -- fa_fp32_ref.py:82-126: per request, S = q k^T * scale,
                        512-column online softmax (hm = max(lm, gm_old),
                        dm = exp(gm_old - hm), ls = exp(S - hm), P = bf16_RNE(ls),
                        gl = dm*gl + rowsum(ls) unquantised, acc = dm*acc + P V),
                        O = acc / gl, LSE = ln(gl) + hm; GQA head h reads kv head
                        h // (H / KVH) (fa_fp32_ref.py:102).
* ``stage1_tieband`` -- fa_fp32_ref.py:150-206: the same plus the per-element bound
                        A of bf16 near-tie rounding flips (kernel gate |O - O_ref| <= A + floor).
                        One deliberate difference: a chunk's ambiguity is decayed by every
                        later running-max step (amb = dm*amb + X, as acc is), where
                        fa_fp32_ref.py:200-201 scales it by its own step only
                        (amb += dm*X), which is not a bound once the max moves. Pinned by
                        brute force over all rounding flips (test_oracle_attention.py).
* ``stage1_rowwise`` -- fa_fp32_ref.py:209-245: scalar per-row loop (cross-check).
* ``pack_lse``       -- the padded LSE layout: row (t*H + h) of 8 identical fp32
                        (.../block_epilogue_rescale_o_no_split_row.hpp:409-416,
                        run_precision_suite.py:72-75).
* ``suffix``         -- per-sequence decode attention (q_len 1, own block-table row,
                        kv length 0 allowed -> O = 0, LSE = -inf). Same arithmetic as
                        ``stage1``; the reference's stage 2 is the closed CANN FIA v2,
                        so parity with it is unpinned.
* ``dense``          -- textbook softmax attention over explicit K/V (the check that
                        pins the chunked forms; BASELINE config 1's criterion).
"""
import numpy as np

from .bf16 import round_bf16

BLOCK_SIZE = 128
CHUNK = 512


def gather_kv(k, v, bt_row, kv):
    """One request's logical K/V [kv, KVH, D] gathered through its block-table row."""
    nblk = (kv + BLOCK_SIZE - 1) // BLOCK_SIZE
    pages = np.asarray(bt_row[:nblk], dtype=np.int64)
    kh = k[pages].reshape(nblk * BLOCK_SIZE, *k.shape[2:])[:kv]
    vh = v[pages].reshape(nblk * BLOCK_SIZE, *v.shape[2:])[:kv]
    return kh, vh


def _q_offsets(q_seqlens):
    return np.concatenate([[0], np.cumsum(np.asarray(q_seqlens, dtype=np.int64))])


def stage1(q, k, v, block_table, q_seqlens, kv_seqlens, chunk=CHUNK, quantize_p=True,
           scale=None, tieband=False, tie_band_rel=2e-5):
    """Stage-1 paged attention, fp64.

    q [T,H,D], k/v [numBlocks,128,KVH,D] (any float dtype holding the bf16 values),
    block_table [B,cols] int, q_seqlens/kv_seqlens [B].
    Returns (O [T,H,D] fp64, LSE [T,H] fp64) and, with ``tieband``, A [T,H,D].

    Query head h reads kv head h // (H / KVH) (fa_fp32_ref.py:102); the products
    run per kv head over its group of query heads (batched BLAS), and requests
    that read the same pages with the same kv length are computed together.
    Every query row is independent, so neither changes the arithmetic.
    """
    q64 = np.asarray(q, dtype=np.float64)
    T, H, D = q64.shape
    KVH = k.shape[2]
    group = H // KVH
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(float(D))))
    O = np.zeros((T, H, D))
    LSE = np.full((T, H), -np.inf)
    A = np.zeros((T, H, D)) if tieband else None
    offs = _q_offsets(q_seqlens)
    work = {}
    for b in range(len(q_seqlens)):
        kv = int(kv_seqlens[b])
        t0, t1 = int(offs[b]), int(offs[b + 1])
        if t1 == t0 or kv <= 0:
            continue
        nblk = (kv + BLOCK_SIZE - 1) // BLOCK_SIZE
        pages = np.asarray(block_table[b][:nblk], dtype=np.int64)
        key = (kv, pages.tobytes())
        work.setdefault(key, (pages, []))[1].append(np.arange(t0, t1))
    for (kv, _), (pages, toks) in work.items():
        rows = np.concatenate(toks)
        Tg = len(rows)
        kb, vb = gather_kv(k, v, pages, kv)
        kb = np.asarray(kb, dtype=np.float64).transpose(1, 2, 0)   # [KVH, D, kv]
        vb = np.asarray(vb, dtype=np.float64).transpose(1, 0, 2)   # [KVH, kv, D]
        # [KVH, group * Tg, D]: row (a, t) is query head g * group + a of token rows[t]
        qb = q64[rows].reshape(Tg, KVH, group, D).transpose(1, 2, 0, 3).reshape(KVH, group * Tg, D)
        m = np.full((KVH, group * Tg), -np.inf)
        gl = np.zeros((KVH, group * Tg))
        acc = np.zeros((KVH, group * Tg, D))
        amb = np.zeros((KVH, group * Tg, D)) if tieband else None
        step = kv if chunk is None else chunk
        for s in range(0, kv, step):
            e = min(kv, s + step)
            sc = np.matmul(qb, kb[:, :, s:e]) * scale
            m_new = np.maximum(m, sc.max(axis=2))
            dm = np.exp(m - m_new) if s > 0 else np.ones_like(m_new)
            ls = np.exp(sc - m_new[:, :, None])
            p = round_bf16(ls).astype(np.float64) if quantize_p else ls
            gl = dm * gl + ls.sum(axis=2)
            acc = dm[:, :, None] * acc + np.matmul(p, vb[:, s:e])
            if tieband:
                amb = dm[:, :, None] * amb + np.matmul(_tie_ambiguity(ls, tie_band_rel), np.abs(vb[:, s:e]))
            m = m_new

        def unfold(x):  # [KVH, group * Tg, ...] -> [Tg, H, ...]
            x = x.reshape(KVH, group, Tg, *x.shape[2:])
            return np.moveaxis(x, 2, 0).reshape(Tg, H, *x.shape[3:])
        O[rows] = unfold(acc / gl[:, :, None])
        LSE[rows] = unfold(np.log(gl) + m)
        if tieband:
            A[rows] = unfold(amb / gl[:, :, None])
    if tieband:
        return O, LSE, A
    return O, LSE


def _tie_ambiguity(ls, tie_band_rel):
    """Width of the bf16 grid interval around ls where |ls - midpoint| is within the
    fp32 S-noise band, else 0 (fa_fp32_ref.py:129-147, 195-200)."""
    x32 = np.asarray(ls, dtype=np.float32)
    u = x32.view(np.uint32).astype(np.uint64)
    rne = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1)))
           & np.uint64(0xFFFF0000))
    p = rne.astype(np.uint32).view(np.float32).astype(np.float64)
    up = (rne + np.uint64(1 << 16)).astype(np.uint32).view(np.float32).astype(np.float64)
    dn = (rne - np.uint64(1 << 16)).astype(np.uint32).view(np.float32).astype(np.float64)
    g_hi = np.where(p < ls, up, p)
    g_lo = np.where(p < ls, p, dn)
    mid = (g_lo + g_hi) / 2.0
    ambiguous = np.abs(ls - mid) <= tie_band_rel * ls
    return ambiguous * (g_hi - g_lo)


def stage1_tieband(q, k, v, block_table, q_seqlens, kv_seqlens, chunk=CHUNK, tie_band_rel=2e-5):
    """(O, LSE, A) with A the near-tie bound of fa_fp32_ref.py:150-206."""
    return stage1(q, k, v, block_table, q_seqlens, kv_seqlens, chunk=chunk, tieband=True,
                  tie_band_rel=tie_band_rel)


def stage1_rowwise(q, k, v, block_table, q_seqlens, kv_seqlens, chunk=CHUNK):
    """Scalar per-(token, head) loop restating fa_fp32_ref.py:209-245 (small cases only)."""
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    v64 = np.asarray(v, dtype=np.float64)
    T, H, D = q64.shape
    group = H // k64.shape[2]
    scale = float(np.float32(1.0 / np.sqrt(float(D))))
    O = np.zeros((T, H, D))
    LSE = np.full((T, H), -np.inf)
    tok = 0
    for b in range(len(q_seqlens)):
        kv = int(kv_seqlens[b])
        kb, vb = gather_kv(k64, v64, block_table[b], kv)
        for tl in range(int(q_seqlens[b])):
            qrow = q64[tok + tl]
            for h in range(H):
                kk, vv = kb[:, h // group, :], vb[:, h // group, :]
                m, gl, acc = -np.inf, 0.0, np.zeros(D)
                for s in range(0, kv, chunk):
                    e = min(kv, s + chunk)
                    sc = (kk[s:e] @ qrow[h]) * scale
                    m_new = max(m, float(sc.max()))
                    dm = np.exp(m - m_new) if s > 0 else 1.0
                    ls = np.exp(sc - m_new)
                    gl = dm * gl + ls.sum()
                    acc = dm * acc + round_bf16(ls).astype(np.float64) @ vv[s:e]
                    m = m_new
                if kv > 0:
                    O[tok + tl, h] = acc / gl
                    LSE[tok + tl, h] = np.log(gl) + m
        tok += int(q_seqlens[b])
    return O, LSE


def pack_lse(lse):
    """[T,H] LSE -> the padded fp32 layout [T*H*8] (8 identical copies per row)."""
    return np.repeat(np.asarray(lse, dtype=np.float32).reshape(-1), 8)


def unpack_lse(lse_padded, T, H):
    """Padded [T*H*8] -> ([T,H] first copies, True if all 8 copies of every row agree)."""
    rows = np.asarray(lse_padded).reshape(T * H, 8)
    same = bool(np.array_equal(rows.view(np.uint32), np.repeat(rows[:, :1], 8, 1).view(np.uint32)))
    return rows[:, 0].reshape(T, H), same


def suffix(q, k, v, block_table, kv_seqlens, chunk=CHUNK):
    """Per-sequence decode attention: q [B,H,D], one query token per sequence.
    Returns (O [B,H,D], LSE [B,H]); kv length 0 gives O = 0, LSE = -inf."""
    B = q.shape[0]
    return stage1(q, k, v, block_table, np.ones(B, dtype=np.int64), kv_seqlens, chunk=chunk)


def dense(q, kh, vh, scale=None):
    """Textbook attention for one query set against explicit K/V.
    q [N,H,D]; kh/vh [S,H,D] (already expanded to query heads). fp64.
    Returns (O [N,H,D], LSE [N,H])."""
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(kh, dtype=np.float64)
    v64 = np.asarray(vh, dtype=np.float64)
    D = q64.shape[-1]
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(float(D))))
    S = np.einsum('nhd,shd->nhs', q64, k64) * scale
    mx = S.max(axis=2, keepdims=True)
    e = np.exp(S - mx)
    den = e.sum(axis=2, keepdims=True)
    O = np.einsum('nhs,shd->nhd', e / den, v64)
    LSE = (np.log(den) + mx)[..., 0]
    return O, LSE


def expand_heads(x, num_heads):
    """[S,KVH,D] -> [S,H,D] with query head h reading kv head h // (H / KVH)."""
    group = num_heads // x.shape[1]
    return x[:, np.arange(num_heads) // group, :]
