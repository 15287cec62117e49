"""Pins oracle.attention: reference fixtures, dense softmax, closed forms, brute
force, and planted mistakes that the checks must catch."""
import os

import numpy as np
import pytest

from oracle import attention as A
from oracle.bf16 import bits_to_f32, round_bf16
from oracle.inputs import paged_inputs
from oracle.merge import merge_fp64


def _dense_request(q, k, v, bt_row, kv, H):
    kh, vh = A.gather_kv(k, v, bt_row, kv)
    return A.dense(q, A.expand_heads(kh, H), A.expand_heads(vh, H))


def test_gather_closed_form_permuted():
    """logical token j of request b == pool[bt[b, j // 128], j % 128] (ID-encoded pool)."""
    nb, KVH, D = 12, 2, 4
    k = np.zeros((nb, 128, KVH, D))
    k[:, :, :, 0] = np.arange(nb)[:, None, None]
    k[:, :, :, 1] = np.arange(128)[None, :, None]
    k[:, :, :, 2] = np.arange(KVH)[None, None, :]
    rng = np.random.default_rng(3)
    bt = rng.permutation(nb).astype(np.int32).reshape(3, 4)
    for b in range(3):
        kv = 300 + 50 * b
        kb, _ = A.gather_kv(k, k, bt[b], kv)
        j = np.arange(kv)
        assert np.array_equal(kb[:, 0, 0], bt[b, j // 128])
        assert np.array_equal(kb[:, 0, 1], j % 128)
        assert np.array_equal(kb[:, 1, 2], np.ones(kv))
        # planted mistake: indexing pages by the transposed table must disagree
        bad, _ = A.gather_kv(k, k, bt.T.reshape(-1)[4 * b:4 * b + 4], kv)
        assert not np.array_equal(bad[:, 0, 0], kb[:, 0, 0])


@pytest.mark.parametrize("kv", [1, 127, 128, 513, 1100])
def test_unquantized_equals_dense(kv):
    inp = paged_inputs(2, [kv, kv // 2 + 1], 8, 2, seed=kv, q_len=3, permute=True)
    O, L = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], inp["q_seqlens"], inp["kv_seqlens"],
                    chunk=None, quantize_p=False)
    for b in range(2):
        Od, Ld = _dense_request(inp["q"][3 * b:3 * b + 3], inp["k"], inp["v"], inp["block_table"][b],
                                int(inp["kv_seqlens"][b]), 8)
        assert np.abs(O[3 * b:3 * b + 3] - Od).max() < 1e-12
        assert np.abs(L[3 * b:3 * b + 3] - Ld).max() < 1e-12


def test_chunked_quantized_within_bf16_bound_of_dense():
    """P rounding moves O by at most 2^-8 * max|v| (bf16 unit roundoff on each weight)
    and leaves LSE unchanged (row sums use the unrounded p)."""
    inp = paged_inputs(3, [1500, 700, 64], 8, 2, seed=5, permute=True)
    O, L = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], inp["q_seqlens"], inp["kv_seqlens"])
    for b in range(3):
        Od, Ld = _dense_request(inp["q"][b:b + 1], inp["k"], inp["v"], inp["block_table"][b],
                                int(inp["kv_seqlens"][b]), 8)
        vmax = np.abs(inp["v"]).max()
        assert np.abs(O[b:b + 1] - Od).max() <= 2.0 ** -8 * vmax + 1e-12
        assert np.abs(L[b:b + 1] - Ld).max() < 1e-10
    O2, L2 = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], inp["q_seqlens"], inp["kv_seqlens"],
                      quantize_p=False)
    assert np.abs(O - O2).max() > 0  # the quantisation point is real


def test_vectorised_equals_rowwise_bruteforce():
    inp = paged_inputs(2, [700, 130], 4, 2, seed=11, q_len=2, permute=True)
    args = (inp["q"], inp["k"], inp["v"], inp["block_table"], inp["q_seqlens"], inp["kv_seqlens"])
    O1, L1 = A.stage1(*args)
    O2, L2 = A.stage1_rowwise(*args)
    assert np.abs(O1 - O2).max() < 1e-12 and np.abs(L1 - L2).max() < 1e-12


def test_gqa_mapping_and_planted_mistake():
    inp = paged_inputs(1, [300], 8, 2, seed=2)
    O, L = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], inp["q_seqlens"], inp["kv_seqlens"],
                    quantize_p=False, chunk=None)
    kh, vh = A.gather_kv(inp["k"], inp["v"], inp["block_table"][0], 300)
    Od, _ = A.dense(inp["q"], A.expand_heads(kh, 8), A.expand_heads(vh, 8))
    assert np.abs(O - Od).max() < 1e-12
    # planted mistake: head h -> kv head h % KVH (interleaved) must be detected
    wrong = np.arange(8) % 2
    Ow, _ = A.dense(inp["q"], kh[:, wrong], vh[:, wrong])
    assert np.abs(O - Ow).max() > 1e-2


def test_closed_forms_single_and_identical_keys():
    rng = np.random.default_rng(4)
    D = 128
    q = round_bf16(rng.standard_normal((1, 2, D)))
    k = round_bf16(rng.standard_normal((2, 128, 1, D)))
    v = round_bf16(rng.standard_normal((2, 128, 1, D)))
    bt = np.array([[1, 0]], dtype=np.int32)
    scale = float(np.float32(1 / np.sqrt(D)))
    # one kv token: O = v, LSE = s
    O, L = A.stage1(q, k, v, bt, [1], [1])
    assert np.allclose(O[0], v[1, 0, 0][None, :], atol=0, rtol=0)
    assert np.allclose(L[0], (q[0].astype(np.float64) @ k[1, 0, 0].astype(np.float64)) * scale, rtol=1e-14)
    # identical keys over 200 tokens: p = 1 exactly, O = mean(v), LSE = s + ln(200)
    k2 = np.repeat(k[:1, :1], 128, axis=1)
    k2 = np.concatenate([k2, k2])
    O, L = A.stage1(q, k2, v, np.array([[0, 1]], dtype=np.int32), [1], [200])
    vv = np.concatenate([v[0, :, 0], v[1, :72, 0]]).astype(np.float64)
    assert np.abs(O[0] - vv.mean(0)).max() < 1e-12
    s = (q[0].astype(np.float64) @ k[0, 0, 0].astype(np.float64)) * scale
    assert np.abs(L[0] - (s + np.log(200))).max() < 1e-12


def test_lse_padded_layout_roundtrip():
    lse = np.random.default_rng(0).standard_normal((5, 3)).astype(np.float32)
    p = A.pack_lse(lse)
    assert p.shape == (5 * 3 * 8,)
    back, same = A.unpack_lse(p, 5, 3)
    assert same and np.array_equal(back, lse)
    # row (t*H + h): the first copy of row 4 is token 1, head 1
    assert p[4 * 8] == lse[1, 1]


def test_empty_suffix():
    inp = paged_inputs(2, [0, 5], 4, 2, seed=1)
    O, L = A.suffix(inp["q"], inp["k"], inp["v"], inp["block_table"], inp["kv_seqlens"])
    assert np.all(O[0] == 0) and np.all(np.isneginf(L[0])) and np.all(np.isfinite(L[1]))


def test_cascade_equals_dense_over_concat():
    """8 sequences share a 1024-token prefix, suffixes U[64,256],
    H=8, KVH=2, fp16-valued inputs; merge(stage1, suffix) == attention over concat."""
    rng = np.random.default_rng(0)
    B, H, KVH, D, P = 8, 8, 2, 128, 1024
    suf = rng.integers(64, 257, size=B)
    nsb = [(int(s) + 127) // 128 for s in suf]
    nblocks = P // 128 + sum(nsb)
    f16 = lambda x: np.asarray(x, dtype=np.float16).astype(np.float64)
    k = f16(rng.standard_normal((nblocks, 128, KVH, D)))
    v = f16(rng.standard_normal((nblocks, 128, KVH, D)))
    q = f16(rng.standard_normal((B, H, D)))
    perm = rng.permutation(nblocks).astype(np.int32)
    bt_pre = perm[:P // 128][None, :]
    bt_suf = np.zeros((B, max(nsb)), dtype=np.int32)
    off = P // 128
    for b in range(B):
        bt_suf[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    O1, L1 = A.stage1(q, k, v, bt_pre, [B], [P])
    O2, L2 = A.suffix(q, k, v, bt_suf, suf)
    Om, Lm = merge_fp64(O1, O2, L1, L2)
    for b in range(B):
        kp, vp = A.gather_kv(k, v, bt_pre[0], P)
        ks, vs = A.gather_kv(k, v, bt_suf[b], int(suf[b]))
        Od, Ld = A.dense(q[b:b + 1], A.expand_heads(np.concatenate([kp, ks]), H),
                         A.expand_heads(np.concatenate([vp, vs]), H))
        assert np.abs(Om[b:b + 1] - Od).max() < 2.0 ** -8 * np.abs(v).max()
        assert np.abs(Lm[b:b + 1] - Ld).max() < 1e-10


def _catlass_inputs(golden_dir):
    d = os.path.join(golden_dir, "catlass_example")
    q = bits_to_f32(np.fromfile(os.path.join(d, "q.bin"), dtype=np.uint16)).reshape(4, 40, 128)
    bt = np.fromfile(os.path.join(d, "block_table.bin"), dtype=np.int32).reshape(4, 32)
    kvs = np.fromfile(os.path.join(d, "kv_seqlen.bin"), dtype=np.int64)
    qs = np.fromfile(os.path.join(d, "q_seqlen.bin"), dtype=np.int64)
    lse = np.fromfile(os.path.join(d, "golden_gpu_lse.bin"), dtype=np.float32).reshape(4, 40)
    return q, bt, qs, kvs, lse


def test_catlass_fixture_lse_statistics(golden_dir):
    """The reference's example-23 fixture: q.bin is U(-1,1); its K/V are missing, so
    K/V are drawn U(-1,1) here. The golden per-row LSE then agrees with the oracle
    in mean (to sampling noise ~5e-4) and spread; a wrong scale (1/128 instead of
    1/sqrt(128)) is off by 0.055, a log2 in place of ln by > 1."""
    q, bt, qs, kvs, lse_g = _catlass_inputs(golden_dir)
    assert np.array_equal(bt, np.arange(128, dtype=np.int32).reshape(4, 32))
    rng = np.random.default_rng(0)
    k = round_bf16(rng.uniform(-1, 1, (128, 128, 8, 128)))
    v = round_bf16(rng.uniform(-1, 1, (128, 128, 8, 128)))
    O, L = A.stage1(q, k, v, bt, qs, kvs)
    assert abs(L.mean() - lse_g.mean()) < 3e-3
    assert 0.5 < L.std() / lse_g.std() < 2.0
    assert np.abs(L - lse_g).max() < 0.05
    g_o = np.fromfile(os.path.join(golden_dir, "catlass_example", "golden_gpu.bin"), dtype=np.float32)
    assert 0.7 < O.std() / g_o.std() < 1.4
    # planted mistakes
    _, Lw = A.stage1(q, k, v, bt, qs, kvs, scale=1.0 / 128)
    assert abs(Lw.mean() - lse_g.mean()) > 0.03
    assert abs((L / np.log(2.0)).mean() - lse_g.mean()) > 1.0  # log2 instead of ln


def test_tie_ambiguity_midpoint_far_and_band_edge():
    """_tie_ambiguity: an ls sitting on a bf16 rounding midpoint is ambiguous by the
    grid spacing there; an ls on the grid or a quarter-spacing away is not; the
    band edge is tie_band_rel * ls (fa_fp32_ref.py:129-147, 195-200)."""
    mid1 = 1.0 + 2.0 ** -8           # between 1 and 1 + 2^-7 (spacing 2^-7 in [1, 2))
    mid2 = 0.3125 + 2.0 ** -10       # between 0.3125 and 0.3125 + 2^-9 (spacing in [0.25, 0.5))
    mid3 = 3.0 + 2.0 ** -7           # between 3 and 3 + 2^-6
    got = A._tie_ambiguity(np.array([mid1, mid2, mid3]), 2e-5)
    assert np.array_equal(got, [2.0 ** -7, 2.0 ** -9, 2.0 ** -6])
    far = np.array([1.0, 1.0 + 2.0 ** -9, 0.3125, 3.0 - 2.0 ** -8])
    assert np.all(A._tie_ambiguity(far, 2e-5) == 0)
    inside = mid1 * (1 - 1e-5)
    outside = mid1 * (1 - 5e-5)
    assert A._tie_ambiguity(np.array([inside]), 2e-5)[0] == 2.0 ** -7
    assert A._tie_ambiguity(np.array([outside]), 2e-5)[0] == 0


def _flip_closed_form(s, v, chunk, flips):
    """O of one query row when the P elements in `flips` take the other bf16 neighbour
    of exp(s - m) instead of the nearest one. Closed form of the chunked online
    softmax: O = sum_i P_i v_i exp(m_c(i) - m_end) / sum_i exp(s_i - m_end), with
    m_c the running max after chunk c; no recurrence shared with the oracle."""
    n = len(s)
    m_after = np.array([s[:min(n, (i // chunk + 1) * chunk)].max() for i in range(n)])
    m_end = s.max()
    ls = np.exp(s - m_after)
    p = round_bf16(ls).astype(np.float64)
    x32 = ls.astype(np.float32).view(np.uint32).astype(np.int64)
    rne = (x32 + 0x7FFF + ((x32 >> 16) & 1)) & 0xFFFF0000
    hi = ((rne + (1 << 16)) & 0xFFFFFFFF).astype(np.uint32).view(np.float32).astype(np.float64)
    lo = ((rne - (1 << 16)) & 0xFFFFFFFF).astype(np.uint32).view(np.float32).astype(np.float64)
    other = np.where(p < ls, hi, lo)
    pp = np.where(flips, other, p)
    gl = np.exp(s - m_end).sum()
    return float((pp * v * np.exp(m_after - m_end)).sum() / gl)


def test_stage1_tieband_bound_is_exact_over_all_flips():
    """Brute force over every subset of rounding flips of a 6-token row in three
    2-token chunks whose max moves twice: with V > 0 and every element ambiguous
    (tie_band_rel = 1), A equals the spread max - min of the flipped outputs and
    bounds each |O_flip - O|. The running-max decay of earlier chunks matters: the
    accumulation sum_s dm_s X_s (each chunk scaled by its own step's decay only)
    misses that spread, which is how the planted mistake is caught."""
    import itertools
    s = np.array([0.0, -1.0, 0.5, 0.2, 2.0, 1.0])
    vv = np.array([1.0, 2.0, 0.5, 3.0, 1.5, 0.25])
    k = np.zeros((1, 128, 1, 1))
    v = np.zeros((1, 128, 1, 1))
    k[0, :6, 0, 0] = s
    v[0, :6, 0, 0] = vv
    q = np.ones((1, 1, 1))
    bt = np.zeros((1, 1), dtype=np.int32)
    O, L, Amb = A.stage1_tieband(q, k, v, bt, [1], [6], chunk=2, tie_band_rel=1.0)
    base = _flip_closed_form(s, vv, 2, np.zeros(6, bool))
    assert abs(base - O[0, 0, 0]) < 1e-14
    deltas = [_flip_closed_form(s, vv, 2, np.array(f, bool)) - base
              for f in itertools.product([0, 1], repeat=6)]
    spread = max(deltas) - min(deltas)
    assert max(abs(d) for d in deltas) <= Amb[0, 0, 0] + 1e-15
    assert abs(spread - Amb[0, 0, 0]) < 1e-14 * max(1.0, spread)
    # planted mistake: each chunk's ambiguity scaled only by its own dm
    m = -np.inf
    gl, wrong = 0.0, 0.0
    for c in range(3):
        sc = s[2 * c:2 * c + 2]
        m_new = max(m, sc.max())
        dm = np.exp(m - m_new) if c else 1.0
        ls = np.exp(sc - m_new)
        gl = dm * gl + ls.sum()
        wrong += dm * (A._tie_ambiguity(ls, 1.0) * vv[2 * c:2 * c + 2]).sum()
        m = m_new
    assert abs(wrong / gl - spread) > 1e-4
    # with the reference's band (2e-5) none of these six is near a tie: A = 0
    _, _, A0 = A.stage1_tieband(q, k, v, bt, [1], [6], chunk=2)
    assert np.all(A0 == 0)
