"""torch CPU restatement of the cascade-decode path -- TEST INFRASTRUCTURE ONLY.

The CPU baseline ``bench.py`` times beside the GPU numbers (its ``cpu_baseline``
leg is the only caller). It computes what the numpy oracle computes, in fp32 with
torch's multithreaded CPU kernels, the way the reference's CPU golden path would
run on the host:

* ``stage1``  -- fa_fp32_ref.py:82-126: per kv head, S = q k^T * scale over
                 512-column chunks, online softmax with P rounded to bf16 (RNE,
                 torch's cast), row sums of the unrounded p, O = acc / l,
                 LSE = ln(l) + m; query head h reads kv head h // (H / KVH).
* ``suffix``  -- the same per sequence over its own pages (q_len 1), unrounded P
                 (this build's stage-2 keeps P in fp32); kv length 0 gives O = 0,
                 LSE = -inf.
* ``merge``   -- lse_merge_cases.py:45-50: m = max, w = exp(l - m), out =
                 (o1 w1 + o2 w2) / (w1 + w2), lse = m + ln(w1 + w2).
* ``swiglu``  -- f3_floor/design.md:107-109: silu(x Wg^T) * (x Wu^T) via F.linear.

Pinned against the numpy oracle (fp64) on small inputs in
``tests/test_oracle_torch_cpu.py``.
"""
import math

import torch
import torch.nn.functional as F

PAGE = 128
CHUNK = 512


def gather(pool, bt_row, kv):
    """[kv, KVH, D] rows of a [nb, 128, KVH, D] pool through one block-table row."""
    nblk = (kv + PAGE - 1) // PAGE
    pages = bt_row[:nblk].long()
    return pool.index_select(0, pages).reshape(nblk * PAGE, *pool.shape[2:])[:kv]


def _attend(qg, kh, vh, scale, chunk, quantize_p):
    """qg [KVH, R, D] fp32 against kh/vh [kv, KVH, D]; returns (O [KVH, R, D], LSE [KVH, R])."""
    kv = kh.shape[0]
    kt = kh.permute(1, 2, 0).float()       # [KVH, D, kv]
    vt = vh.permute(1, 0, 2).float()       # [KVH, kv, D]
    G, R, D = qg.shape
    m = torch.full((G, R), -math.inf)
    gl = torch.zeros(G, R)
    acc = torch.zeros(G, R, D)
    step = kv if chunk is None else chunk
    for s in range(0, kv, step):
        e = min(kv, s + step)
        sc = torch.bmm(qg, kt[:, :, s:e]) * scale
        m_new = torch.maximum(m, sc.amax(dim=2))
        dm = torch.exp(m - m_new) if s > 0 else torch.ones_like(m_new)
        ls = torch.exp(sc - m_new[:, :, None])
        p = ls.to(torch.bfloat16).float() if quantize_p else ls
        gl = dm * gl + ls.sum(dim=2)
        acc = dm[:, :, None] * acc + torch.bmm(p, vt[:, s:e])
        m = m_new
    return acc / gl[:, :, None], torch.log(gl) + m


def stage1(q, k, v, bt_row, kv, scale=None, chunk=CHUNK):
    """All T queries of q [T, H, D] against one request's kv tokens (the flattened
    shared-prefix form). Returns (O [T, H, D] fp32, LSE [T, H] fp32)."""
    T, H, D = q.shape
    KVH = k.shape[2]
    grp = H // KVH
    scale = scale if scale is not None else float(torch.tensor(1.0 / math.sqrt(D), dtype=torch.float32))
    qg = q.float().reshape(T, KVH, grp, D).permute(1, 2, 0, 3).reshape(KVH, grp * T, D)
    O, L = _attend(qg, gather(k, bt_row, kv), gather(v, bt_row, kv), scale, chunk, True)
    O = O.reshape(KVH, grp, T, D).permute(2, 0, 1, 3).reshape(T, H, D)
    L = L.reshape(KVH, grp, T).permute(2, 0, 1).reshape(T, H)
    return O, L


def suffix(q, k, v, block_table, kv_seqlens, scale=None):
    """Per-sequence decode: q [B, H, D], sequence b over its own block-table row.
    Returns (O [B, H, D] fp32, LSE [B, H] fp32)."""
    B, H, D = q.shape
    KVH = k.shape[2]
    grp = H // KVH
    scale = scale if scale is not None else float(torch.tensor(1.0 / math.sqrt(D), dtype=torch.float32))
    O = torch.zeros(B, H, D)
    L = torch.full((B, H), -math.inf)
    for b in range(B):
        kv = int(kv_seqlens[b])
        if kv <= 0:
            continue
        qg = q[b].float().reshape(KVH, grp, D)
        o, l = _attend(qg, gather(k, block_table[b], kv), gather(v, block_table[b], kv), scale, CHUNK, False)
        O[b] = o.reshape(H, D)
        L[b] = l.reshape(H)
    return O, L


def merge(o1, o2, l1, l2):
    """Two partial results [..., D] with LSEs [...] -> (out, lse). A side at -inf
    has weight 0; both at -inf give out = 0, lse = -inf."""
    m = torch.maximum(l1, l2)
    mu = torch.where(torch.isinf(m) & (m < 0), torch.zeros_like(m), m)
    w1 = torch.exp(l1 - mu)
    w2 = torch.exp(l2 - mu)
    s = w1 + w2
    inv = torch.where(s > 0, 1.0 / s, torch.zeros_like(s))
    out = (o1.float() * w1[..., None] + o2.float() * w2[..., None]) * inv[..., None]
    lse = torch.where(s > 0, mu + torch.log(s), torch.full_like(s, -math.inf))
    return out, lse


def swiglu(a, w):
    """a [M, K], w [2I, K] (gate rows then up rows) -> silu(a Wg^T) * (a Wu^T) [M, I], fp32."""
    n_half = w.shape[0] // 2
    c = F.linear(a.float(), w.float())
    return F.silu(c[:, :n_half]) * c[:, n_half:]
