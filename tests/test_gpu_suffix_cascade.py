"""GPU parity of suffix_decode (stage 2) and of the full cascade (stage 1 + suffix
+ merge) against the oracle and dense attention over the concatenated KV.

suffix_decode keeps P at fp32 precision (on the matrix cores as two bf16 terms whose sum is P within
2^-16 P), so its oracle is the unquantised online softmax.
Its O is bf16: the tolerance is the north-star 2e-3 plus half a bf16 ulp of |O|.
"""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.bf16 import bits_to_f32, bf16_bits
from oracle.inputs import paged_inputs
from oracle.merge import merge_fp64
from tests._util import bf16_to_np, torch_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("no_wait_giveups")]
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import cascade_amd  # noqa: F401
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def _suffix(inp):
    q = torch_bf16(inp["q16"], DEV)
    k = torch_bf16(inp["k16"], DEV)
    v = torch_bf16(inp["v16"], DEV)
    bt = torch.from_numpy(inp["block_table"]).to(DEV)
    kvs = torch.from_numpy(inp["kv_seqlens"]).to(DEV)
    out, lse = torch.ops.npu.suffix_decode(q, k, v, bt, kvs)
    torch.cuda.synchronize()
    return bf16_to_np(out), lse.cpu().numpy()


def _check_suffix(inp, out, lse, H):
    B = inp["q"].shape[0]
    O_ref, L_ref = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], np.ones(B, dtype=np.int64),
                            inp["kv_seqlens"], quantize_p=False)
    L = lse.reshape(B, H)
    err = np.abs(out - O_ref)
    assert np.all(err <= 2e-3 + 2.0 ** -8 * np.abs(O_ref)), err.max()
    fin = np.isfinite(L_ref)
    assert np.array_equal(np.isfinite(L), fin)
    assert np.all(np.isneginf(L[~fin]))
    assert np.all(out[~fin] == 0)
    if fin.any():
        rel = np.abs(L[fin] - L_ref[fin]) / np.maximum(np.abs(L_ref[fin]), 1.0)
        assert rel.max() <= 1e-4, rel.max()


SUFFIX_CASES = [
    ("decode_b8_h32", 8, [1, 2, 63, 64, 65, 127, 128, 300], 32, 8),
    ("empty_and_short", 6, [0, 1, 0, 17, 200, 0], 16, 4),
    ("long_multi_split", 3, [3000, 4096, 513], 32, 8),
    ("gqa8_h64", 5, [700, 90, 1025, 2, 4000], 64, 8),
    ("mha_h8_kvh8", 4, [100, 200, 300, 400], 8, 8),
    ("group2", 4, [257, 33, 1000, 5], 8, 4),
    # more than 8 query heads per kv head: split into groups of <= 8 that share the kv head
    ("gqa16_h64_kvh4", 5, [700, 0, 1025, 64, 3000], 64, 4),
    ("gqa12_h48_kvh4", 3, [129, 2000, 1], 48, 4),
    ("gqa11_h11_kvh1", 3, [500, 77, 1300], 11, 1),
    # odd group sizes: the matrix-core body's padding heads (columns G .. 15)
    ("gqa3_h12_kvh4", 5, [1, 300, 65, 0, 1500], 12, 4),
    ("gqa5_h20_kvh4", 4, [129, 2000, 7, 640], 20, 4),
    ("gqa7_h28_kvh4", 3, [900, 33, 257], 28, 4),
]


@pytest.mark.parametrize("case", SUFFIX_CASES, ids=[c[0] for c in SUFFIX_CASES])
def test_suffix_cases(case):
    name, B, kvs, H, KVH = case
    inp = paged_inputs(B, kvs, H, KVH, seed=len(name), permute=True)
    out, lse = _suffix(inp)
    _check_suffix(inp, out, lse, H)


def test_suffix_geometric_lengths():
    """BASELINE config 5's suffix distribution (geometric, mean 512, clipped to
    [1, 4096]) at a reduced batch."""
    rng = np.random.default_rng(1)
    B, H, KVH = 24, 64, 8
    kvs = np.clip(rng.geometric(1 / 512, size=B), 1, 4096)
    inp = paged_inputs(B, kvs, H, KVH, seed=2, permute=True, block_cols=32)
    out, lse = _suffix(inp)
    _check_suffix(inp, out, lse, H)


def _stand_alone_chunk_segments(kvs, num_heads, kv_heads):
    """Most sequences any chunk of the stand-alone suffix grid holds (host
    restatement: 32-token windows, 512 / kv head groups equal chunks)."""
    groups = kv_heads * ((num_heads // kv_heads + 7) // 8)
    P = max(512 // groups, 1)
    wins = [(int(x) + 31) // 32 for x in kvs]
    cw = np.concatenate([[0], np.cumsum(wins)])
    W = int(cw[-1])
    most = 0
    for c in range(P):
        c0, c1 = c * W // P, (c + 1) * W // P
        most = max(most, sum(1 for b in range(len(kvs)) if cw[b + 1] > cw[b] and cw[b] < c1 and cw[b + 1] > c0))
    return most


@pytest.mark.parametrize("B,H,KVH,seed", [(768, 32, 8, 11), (640, 64, 8, 12)], ids=["g4_b768", "g8_b640"])
def test_suffix_chunks_spanning_table_phases(B, H, KVH, seed):
    """Hundreds of short suffixes (1-20 tokens, some empty): stand-alone chunks hold
    more than the 8 sequences of one table phase, so the matrix-core stream body
    crosses phase boundaries at 4 and at 8 query heads per group."""
    rng = np.random.default_rng(seed)
    kvs = rng.integers(1, 21, size=B)
    kvs[rng.random(B) < 0.1] = 0
    assert _stand_alone_chunk_segments(kvs, H, KVH) > 8  # the premise: chunks span phases
    inp = paged_inputs(B, kvs, H, KVH, seed=seed, permute=True)
    out, lse = _suffix(inp)
    _check_suffix(inp, out, lse, H)


def test_suffix_abi_matches_torch_op():
    from cascade_amd import abi
    inp = paged_inputs(4, [1500, 10, 0, 900], 32, 8, seed=3, permute=True)
    q = torch_bf16(inp["q16"], DEV)
    k = torch_bf16(inp["k16"], DEV)
    v = torch_bf16(inp["v16"], DEV)
    bt = torch.from_numpy(inp["block_table"]).to(DEV)
    kvs = torch.from_numpy(inp["kv_seqlens"]).to(DEV)
    cap = bt.shape[1] * 128
    s, wsb = abi.suffix_plan(4, 32, 8, 128, cap)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    out = torch.empty(4, 32, 128, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(4 * 32, dtype=torch.float32, device=DEV)
    rc = abi.lib().ck_suffix_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), bt.shape[1],
                                    kvs.data_ptr(), 4, 32, 8, 128, k.shape[0], 128, abi.CK_KV_NHD,
                                    float(np.float32(1 / np.sqrt(128))), cap, s, out.data_ptr(), lse.data_ptr(),
                                    ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    abi.check(rc)
    o2, l2 = torch.ops.npu.suffix_decode(q, k, v, bt, kvs)
    assert torch.equal(out, o2) and torch.equal(lse, l2)


def _cascade_inputs(B, H, KVH, P, suf, seed):
    rng = np.random.default_rng(seed)
    nsb = [(int(s) + 127) // 128 for s in suf]
    nblocks = P // 128 + sum(nsb)
    k = rng.standard_normal((nblocks, 128, KVH, 128)).astype(np.float32)
    v = rng.standard_normal((nblocks, 128, KVH, 128)).astype(np.float32)
    q = rng.standard_normal((B, H, 128)).astype(np.float32)
    perm = rng.permutation(nblocks).astype(np.int32)
    bt_pre = perm[:P // 128][None, :].copy()
    bt_suf = np.zeros((B, max(max(nsb), 1)), dtype=np.int32)
    off = P // 128
    for b in range(B):
        bt_suf[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    return bf16_bits(q), bf16_bits(k), bf16_bits(v), bt_pre, bt_suf, np.asarray(suf, dtype=np.int64)


CASCADE_CFGS = [
    (8, 8, 2, 1024, "u64_256"),      # BASELINE config 1 shape
    (16, 32, 8, 2048, "geo512"),
    (4, 32, 8, 512, "with_empty"),
    (6, 64, 8, 640, "long_cut"),     # G = 8; suffixes cut across workgroups
    (40, 16, 2, 0, "no_prefix"),     # empty prefix: the suffix alone
    (3, 8, 8, 256, "all_empty"),     # every suffix empty: the prefix alone
    (6, 64, 4, 640, "long_cut"),     # 16 query heads per kv head: two kv head groups
    (10, 6, 2, 512, "geo512"),       # G = 3, 2 and 1 with suffixes: the fused matrix-core body's padding heads
    (4, 4, 2, 384, "with_empty"),
    (9, 8, 8, 256, "geo512"),
    (8, 14, 2, 512, "geo512"),       # G = 7: the fused kernel's dims-major streaming waves
]
CASCADE_IDS = ["config1_b8_h8", "b16_h32_geo", "empty_suffix", "gqa8_long_cut", "empty_prefix", "all_suffix_empty",
               "gqa16_long_cut", "gqa3_geo", "gqa2_with_empty", "mha_geo", "gqa7_geo"]
# the three-op composition cannot take an empty prefix: fa_fp32_stage1 requires kv
# seqlens >= 1 (the reference's op_host contract), so that case runs fused only
CASCADE_RUNS = [(cfg, fused) for cfg in CASCADE_CFGS for fused in (True, False) if fused or cfg[3] > 0]
CASCADE_RUN_IDS = ["%s-%s" % (CASCADE_IDS[CASCADE_CFGS.index(c)], "fused" if f else "unfused")
                   for c, f in CASCADE_RUNS]


def _cascade_case(cfg):
    B, H, KVH, P, dist = cfg
    rng = np.random.default_rng(B)
    if dist == "u64_256":
        suf = rng.integers(64, 257, size=B)
    elif dist == "geo512":
        suf = np.clip(rng.geometric(1 / 512, size=B), 1, 4096)
    elif dist == "with_empty":
        suf = np.array([0, 5, 0, 300])
    elif dist == "long_cut":
        suf = np.array([4000, 1, 2500, 129, 3333, 64])
    elif dist == "no_prefix":
        suf = rng.integers(0, 300, size=B)
    else:
        suf = np.zeros(B, dtype=np.int64)
    return (B, H, KVH, P) + _cascade_inputs(B, H, KVH, P, suf, seed=B)


def _cascade_run(fused, B, P, q, k, v, bt_pre, bt_suf, suf):
    import cascade_amd
    bt_pre_t = torch.from_numpy(bt_pre if bt_pre.shape[1] else np.zeros((1, 1), np.int32)).to(DEV)
    plen = torch.tensor([P], dtype=torch.int64, device=DEV)
    args = (q, k, v, bt_pre_t, plen, k, v, torch.from_numpy(bt_suf).to(DEV), torch.from_numpy(suf).to(DEV))
    if fused:
        out, lse = cascade_amd.ops.cascade_decode(*args)
    else:
        out, lse = cascade_amd.ops.cascade_decode_unfused(*args), None
    torch.cuda.synchronize()
    return bf16_to_np(out), (None if lse is None else lse.cpu().numpy())


@pytest.mark.parametrize("cfg,fused", CASCADE_RUNS, ids=CASCADE_RUN_IDS)
def test_cascade_equals_dense_over_concat(cfg, fused):
    """Config 1 shape (and more): cascade decode == softmax attention over the
    concatenated prefix + suffix KV (bf16 output), for the fused op and for the
    reference's three-op composition; the fused op's merged LSE matches too."""
    B, H, KVH, P, q16, k16, v16, bt_pre, bt_suf, suf = _cascade_case(cfg)
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    got, lse = _cascade_run(fused, B, P, q, k, v, bt_pre, bt_suf, suf)
    qf, kf, vf = bits_to_f32(q16), bits_to_f32(k16), bits_to_f32(v16)
    for b in range(B):
        kp, vp = A.gather_kv(kf, vf, bt_pre[0], P) if P else (kf[:0, 0], vf[:0, 0])
        ks, vs = A.gather_kv(kf, vf, bt_suf[b], int(suf[b]))
        kc, vc = np.concatenate([kp, ks]), np.concatenate([vp, vs])
        if kc.shape[0] == 0:
            assert np.all(got[b] == 0)
            if lse is not None:
                assert np.all(np.isneginf(lse.reshape(B, H)[b]))
            continue
        Od, Ld = A.dense(qf[b:b + 1], A.expand_heads(kc, H), A.expand_heads(vc, H))
        err = np.abs(got[b:b + 1] - Od)
        assert np.all(err <= 2e-3 + 2.0 ** -8 * np.abs(Od)), (b, err.max())
        if lse is not None:
            rel = np.abs(lse.reshape(B, H)[b] - Ld[0]) / np.maximum(np.abs(Ld[0]), 1.0)
            assert rel.max() <= 1e-4, (b, rel.max())
    # and equals the oracle's own cascade composition
    if P:
        O1, L1 = A.stage1(qf, kf, vf, bt_pre, [B], [P])
        O2, L2 = A.stage1(qf, kf, vf, bt_suf, np.ones(B, dtype=np.int64), suf, quantize_p=False)
        Om, _ = merge_fp64(O1, O2, L1, L2)
        assert np.all(np.abs(got - Om) <= 2e-3 + 2.0 ** -8 * np.abs(Om))


def test_cascade_fused_matches_unfused():
    """The fused op and the three-op composition differ only by rounding: the
    composition rounds a cut suffix's result to bf16 before the merge."""
    B, H, KVH, P, q16, k16, v16, bt_pre, bt_suf, suf = _cascade_case((16, 32, 8, 2048, "geo512"))
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    a, _ = _cascade_run(True, B, P, q, k, v, bt_pre, bt_suf, suf)
    b, _ = _cascade_run(False, B, P, q, k, v, bt_pre, bt_suf, suf)
    assert np.all(np.abs(a - b) <= 2.0 ** -7 * np.abs(b) + 1e-3)


def test_cascade_two_launch_groups():
    """More sequences than one suffix launch holds (1024): the fused op runs the
    suffix and epilogue per group (three here); every row still matches the
    composition."""
    B, H, KVH, P = 2100, 8, 2, 256
    rng = np.random.default_rng(7)
    suf = rng.integers(0, 80, size=B)
    q16, k16, v16, bt_pre, bt_suf, suf = _cascade_inputs(B, H, KVH, P, suf, seed=7)
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    a, lse = _cascade_run(True, B, P, q, k, v, bt_pre, bt_suf, suf)
    b, _ = _cascade_run(False, B, P, q, k, v, bt_pre, bt_suf, suf)
    assert np.all(np.abs(a - b) <= 2.0 ** -7 * np.abs(b) + 1e-3)
    assert np.all(np.isfinite(lse))


def test_cascade_config5_full_size():
    """BASELINE config 5 at its full size: H = 64, KVH = 8, a 32768-token shared
    prefix, 256 sequences with geometric suffixes (mean 512, clipped to [1, 4096]),
    permuted pages; K/V/q generated on the device. Every row: the fused op equals
    the three-op composition up to the composition's bf16 rounding of the suffix
    result. Sampled sequences (the longest and shortest suffix and two others):
    equal to dense attention over the concatenated KV, which is exact row sampling
    (a sequence's output depends only on its own query, the prefix and its suffix)."""
    import cascade_amd
    B, H, KVH, P = 256, 64, 8, 32768
    rng = np.random.default_rng(55)
    suf = np.clip(rng.geometric(1 / 512, size=B), 1, 4096).astype(np.int64)
    nsb = [(int(x) + 127) // 128 for x in suf]
    nblocks = P // 128 + sum(nsb)
    perm = rng.permutation(nblocks).astype(np.int32)
    bt_pre = perm[:P // 128][None, :].copy()
    bt_suf = np.zeros((B, max(nsb)), dtype=np.int32)
    off = P // 128
    for b in range(B):
        bt_suf[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    g = torch.Generator(device=DEV).manual_seed(55)
    k = torch.randn(nblocks, 128, KVH, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(nblocks, 128, KVH, 128, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    args = (q, k, v, torch.from_numpy(bt_pre).to(DEV), torch.tensor([P], dtype=torch.int64, device=DEV),
            k, v, torch.from_numpy(bt_suf).to(DEV), torch.from_numpy(suf).to(DEV))
    out, lse = cascade_amd.ops.cascade_decode(*args)
    ref3 = cascade_amd.ops.cascade_decode_unfused(*args)
    torch.cuda.synchronize()
    a, c = out.float(), ref3.float()
    assert bool(((a - c).abs() <= 2.0 ** -7 * c.abs() + 1e-3).all())
    assert bool(torch.isfinite(lse).all())

    got = bf16_to_np(out)
    L = lse.cpu().numpy().reshape(B, H)
    qf = bits_to_f32(q.cpu().view(torch.int16).numpy().view(np.uint16))
    pre_pages = torch.from_numpy(bt_pre[0].astype(np.int64)).to(DEV)
    kp = k[pre_pages].reshape(P, KVH, 128).float().cpu().numpy()
    vp = v[pre_pages].reshape(P, KVH, 128).float().cpu().numpy()
    picks = sorted({int(np.argmax(suf)), int(np.argmin(suf)), 17, 200})
    G = H // KVH
    for b in picks:
        pages = torch.from_numpy(bt_suf[b, :nsb[b]].astype(np.int64)).to(DEV)
        ks = k[pages].reshape(-1, KVH, 128)[:suf[b]].float().cpu().numpy()
        vs = v[pages].reshape(-1, KVH, 128)[:suf[b]].float().cpu().numpy()
        kc, vc = np.concatenate([kp, ks]), np.concatenate([vp, vs])
        for kvh in range(KVH):
            hs = slice(kvh * G, (kvh + 1) * G)
            kg = np.repeat(kc[:, kvh:kvh + 1], G, axis=1)
            vg = np.repeat(vc[:, kvh:kvh + 1], G, axis=1)
            Od, Ld = A.dense(qf[b:b + 1, hs], kg, vg)
            err = np.abs(got[b:b + 1, hs] - Od)
            assert np.all(err <= 2e-3 + 2.0 ** -8 * np.abs(Od)), (b, kvh, err.max())
            rel = np.abs(L[b, hs] - Ld[0]) / np.maximum(np.abs(Ld[0]), 1.0)
            assert rel.max() <= 1e-4, (b, kvh, rel.max())


def test_cascade_abi_matches_torch_op():
    """ck_cascade_decode through ctypes == torch.ops.npu.cascade_decode (bitwise)."""
    import cascade_amd
    from cascade_amd import abi
    B, H, KVH, P, q16, k16, v16, bt_pre, bt_suf, suf = _cascade_case((16, 32, 8, 2048, "geo512"))
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    btp = torch.from_numpy(bt_pre).to(DEV)
    bts = torch.from_numpy(bt_suf).to(DEV)
    plen = torch.tensor([P], dtype=torch.int64, device=DEV)
    sl = torch.from_numpy(suf).to(DEV)
    pcap, scap = btp.shape[1] * 128, bts.shape[1] * 128
    wsb = abi.cascade_plan(B, H, KVH, 128, pcap, scap)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    out = torch.empty(B, H, 128, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(B * H, dtype=torch.float32, device=DEV)
    rc = abi.lib().ck_cascade_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), btp.data_ptr(), btp.shape[1],
                                     plen.data_ptr(), k.shape[0], k.data_ptr(), v.data_ptr(), bts.data_ptr(),
                                     bts.shape[1], sl.data_ptr(), k.shape[0], abi.CK_KV_NHD, B, H, KVH, 128, 128,
                                     float(np.float32(1 / np.sqrt(128.0))), pcap, scap, out.data_ptr(),
                                     lse.data_ptr(), ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    abi.check(rc)
    o2, l2 = cascade_amd.ops.cascade_decode(q, k, v, btp, plen, k, v, bts, sl)
    torch.cuda.synchronize()
    assert torch.equal(out, o2) and torch.equal(lse, l2)
    # a short workspace is refused before anything is launched
    assert abi.lib().ck_cascade_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), btp.data_ptr(), btp.shape[1],
                                       plen.data_ptr(), k.shape[0], k.data_ptr(), v.data_ptr(), bts.data_ptr(),
                                       bts.shape[1], sl.data_ptr(), k.shape[0], abi.CK_KV_NHD, B, H, KVH, 128, 128, 0.088,
                                       pcap, scap, out.data_ptr(), lse.data_ptr(), ws.data_ptr(), wsb - 1,
                                       torch.cuda.current_stream().cuda_stream) == -3


def _bnsd(pool):
    """NHD [nb, 128, KVH, D] -> BNSD [nb, KVH, 128, D] copy of the same pages."""
    return pool.permute(0, 2, 1, 3).contiguous()


@pytest.mark.parametrize("case", SUFFIX_CASES[:4], ids=[c[0] for c in SUFFIX_CASES[:4]])
def test_suffix_bnsd_layout_matches_nhd(case):
    """The BNSD pool layout (the reference's stage-2 input, ascend-kernel/README.md:182-183)
    reads the same rows through other strides: results are bit-identical to NHD."""
    name, B, kvs, H, KVH = case
    inp = paged_inputs(B, kvs, H, KVH, seed=len(name) + 7, permute=True)
    q = torch_bf16(inp["q16"], DEV)
    k = torch_bf16(inp["k16"], DEV)
    v = torch_bf16(inp["v16"], DEV)
    bt = torch.from_numpy(inp["block_table"]).to(DEV)
    kl = torch.from_numpy(inp["kv_seqlens"]).to(DEV)
    o1, l1 = torch.ops.npu.suffix_decode(q, k, v, bt, kl)
    o2, l2 = torch.ops.npu.suffix_decode(q, _bnsd(k), _bnsd(v), bt, kl, 1)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_cascade_bnsd_suffix_pool_matches_nhd():
    import cascade_amd
    B, H, KVH, P, q16, k16, v16, bt_pre, bt_suf, suf = _cascade_case((6, 64, 8, 640, "long_cut"))
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    btp = torch.from_numpy(bt_pre).to(DEV)
    bts = torch.from_numpy(bt_suf).to(DEV)
    plen = torch.tensor([P], dtype=torch.int64, device=DEV)
    sl = torch.from_numpy(suf).to(DEV)
    o1, l1 = cascade_amd.ops.cascade_decode(q, k, v, btp, plen, k, v, bts, sl)
    o2, l2 = cascade_amd.ops.cascade_decode(q, k, v, btp, plen, _bnsd(k), _bnsd(v), bts, sl, 1)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    with pytest.raises(RuntimeError, match="cascade_decode"):
        cascade_amd.ops.cascade_decode(q, k, v, btp, plen, k, v, bts, sl, 2)


@pytest.mark.parametrize("case", [SUFFIX_CASES[1], SUFFIX_CASES[3]], ids=[SUFFIX_CASES[1][0], SUFFIX_CASES[3][0]])
def test_suffix_bnsd_layout_against_oracle(case):
    """A BNSD pool [blocks, KVH, 128, 128] built directly (not copied from an NHD
    pool), called through the C ABI with kv_layout = CK_KV_BNSD and checked against
    the oracle on the same logical K/V."""
    from cascade_amd import abi
    name, B, kvs, H, KVH = case
    inp = paged_inputs(B, kvs, H, KVH, seed=len(name) + 21, permute=True)
    k_bnsd = np.ascontiguousarray(inp["k16"].transpose(0, 2, 1, 3))
    v_bnsd = np.ascontiguousarray(inp["v16"].transpose(0, 2, 1, 3))
    q = torch_bf16(inp["q16"], DEV)
    k = torch_bf16(k_bnsd, DEV)
    v = torch_bf16(v_bnsd, DEV)
    bt = torch.from_numpy(inp["block_table"]).to(DEV)
    kl = torch.from_numpy(inp["kv_seqlens"]).to(DEV)
    cap = bt.shape[1] * 128
    s, wsb = abi.suffix_plan(B, H, KVH, 128, cap)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    out = torch.empty(B, H, 128, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(B * H, dtype=torch.float32, device=DEV)
    rc = abi.lib().ck_suffix_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), bt.shape[1],
                                    kl.data_ptr(), B, H, KVH, 128, k.shape[0], 128, abi.CK_KV_BNSD,
                                    float(np.float32(1 / np.sqrt(128))), cap, s, out.data_ptr(), lse.data_ptr(),
                                    ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    abi.check(rc)
    torch.cuda.synchronize()
    _check_suffix(inp, bf16_to_np(out), lse.cpu().numpy(), H)
