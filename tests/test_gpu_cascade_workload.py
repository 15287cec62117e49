"""GPU parity of the fused cascade at the benchmark's own workload and at batch
shapes whose fused chunks span several table phases.

* The benchmark workload (bench.py's step, BASELINE config 2 end to end): B = 64
  decode queries, H32 / KVH8 / D128, a shared 8192-token prefix over permuted
  pages, 64 suffixes ~Geometric(mean 512) clipped to [1, 4096] with the bench's
  seed (33 787 tokens). This is the launch the headline number times: 8 kv heads
  x 2 m-tiles of 128 rows x 16 prefix splits = 256 stage-1 units beside 256
  suffix chunk pairs. Every one of the 64 x 32 rows is checked against fp64
  softmax attention over the concatenated prefix + suffix KV and against the
  oracle's composition (stage-1 with bf16 P, fp32-P suffix, fp64 merge); ten
  calls in a row must be bit-identical, as the reference requires of stage-1
  (ascend-kernel/csrc/ops/fa_fp32_stage1/test/test_fa_fp32_stage1_smoke.py:110).
  The reference gates its own end-to-end chain at this shape
  (.../fa_fp32_stage1/test/run_merge_probe.py:22,130-138).
* Large batches of short suffixes at 4 query heads per kv head: a fused chunk
  then holds more than 8 sequences (the segment slots of one table phase), so
  the token-major streaming loop crosses phase boundaries inside a chunk.

Tolerances: O max-abs 2e-3 plus half a bf16 ulp of |O| (bf16 output), LSE 1e-4
relative (north star).
"""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.bf16 import bf16_bits, bits_to_f32
from oracle.merge import merge_fp64
from tests._util import bf16_to_np, record_margin, torch_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("no_wait_giveups")]
DEV = "cuda:0"
SCALE = float(np.float32(1.0 / np.sqrt(128.0)))


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import cascade_amd  # noqa: F401
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def bench_suffix_lengths():
    """bench.py's suffix lengths: Geometric(1/512) with seed 0, clipped to [1, 4096]."""
    rng = np.random.default_rng(0)
    return np.clip(rng.geometric(1.0 / 512, size=64), 1, 4096).astype(np.int64)


def _randn_bf16_bits(gen, shape):
    """N(0,1) rounded to bf16 (torch's CPU cast: RNE, the oracle's bf16_bits rule,
    pinned in test_oracle_bf16.py; much faster on pools of ~10^8 elements)."""
    x = torch.randn(*shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16)


def make_inputs(B, H, KVH, P, suf, seed):
    """bf16 q/k/v bit patterns from N(0,1), one pool holding the prefix pages and
    every suffix's own pages, physical pages permuted."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    nsb = [(int(s) + 127) // 128 for s in suf]
    nblocks = P // 128 + sum(nsb)
    k16 = _randn_bf16_bits(gen, (nblocks, 128, KVH, 128))
    v16 = _randn_bf16_bits(gen, (nblocks, 128, KVH, 128))
    q16 = bf16_bits(rng.standard_normal((B, H, 128), dtype=np.float32))
    perm = rng.permutation(nblocks).astype(np.int32)
    bt_pre = perm[:P // 128][None, :].copy()
    bt_suf = np.zeros((B, max(max(nsb), 1)), dtype=np.int32)
    off = P // 128
    for b in range(B):
        bt_suf[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    return q16, k16, v16, bt_pre, bt_suf, np.asarray(suf, dtype=np.int64)


def dense_cascade(qf, kf, vf, bt_pre, P, bt_suf, suf):
    """fp64 softmax attention of every query row over the prefix followed by its
    own suffix, per kv head, with one maximum over the whole concatenated row."""
    B, H, D = qf.shape
    KVH = kf.shape[2]
    G = H // KVH
    kp, vp = A.gather_kv(kf, vf, bt_pre[0], P)
    suf_kv = [A.gather_kv(kf, vf, bt_suf[b], int(suf[b])) for b in range(B)]
    O = np.zeros((B, H, D))
    L = np.zeros((B, H))
    for g in range(KVH):
        hs = slice(g * G, (g + 1) * G)
        qg = qf[:, hs].astype(np.float64)
        kpg = np.ascontiguousarray(kp[:, g], dtype=np.float64)
        vpg = np.ascontiguousarray(vp[:, g], dtype=np.float64)
        sp = (qg.reshape(B * G, D) @ kpg.T).reshape(B, G, -1) * SCALE
        for b in range(B):
            ks, vs = suf_kv[b]
            ss = (qg[b] @ ks[:, g].astype(np.float64).T) * SCALE
            mx = np.maximum(sp[b].max(axis=1) if P else -np.inf, ss.max(axis=1) if ss.shape[1] else -np.inf)
            ep = np.exp(sp[b] - mx[:, None])
            es = np.exp(ss - mx[:, None])
            den = ep.sum(axis=1) + es.sum(axis=1)
            O[b, hs] = (ep @ vpg + es @ vs[:, g].astype(np.float64)) / den[:, None]
            L[b, hs] = np.log(den) + mx
    return O, L


def oracle_cascade(qf, kf, vf, bt_pre, P, bt_suf, suf):
    """The oracle's composition: stage-1 in the flattened form (bf16 P on 512-column
    chunks), the fp32-P suffix, the fp64 LSE merge."""
    B = qf.shape[0]
    O1, L1 = A.stage1(qf, kf, vf, bt_pre, [B], [P])
    O2, L2 = A.stage1(qf, kf, vf, bt_suf, np.ones(B, dtype=np.int64), suf, quantize_p=False)
    return merge_fp64(O1, O2, L1, L2)


def run_cascade(q, k, v, bt_pre, P, bt_suf, suf):
    import cascade_amd
    out, lse = cascade_amd.ops.cascade_decode(q, k, v, torch.from_numpy(bt_pre).to(DEV),
                                              torch.tensor([P], dtype=torch.int64, device=DEV), k, v,
                                              torch.from_numpy(bt_suf).to(DEV), torch.from_numpy(suf).to(DEV))
    return out, lse


def check_rows(name, got, lse, O_ref, L_ref, what):
    err = np.abs(got - O_ref)
    half_ulp = 2.0 ** -8 * np.abs(O_ref)  # the bf16 output's own rounding
    bound = 2e-3 + half_ulp
    rel = np.abs(lse - L_ref) / np.maximum(np.abs(L_ref), 1.0)
    # recorded: the largest error beyond the output rounding, against the 2e-3 tolerance
    record_margin("%s vs %s" % (name, what), np.maximum(err - half_ulp, 0.0).max(), 2e-3, rel.max(), 1e-4)
    assert np.all(err <= bound), (what, err.max(), np.unravel_index(np.argmax(err - bound), err.shape))
    assert rel.max() <= 1e-4, (what, rel.max())


def test_cascade_benchmark_workload():
    B, H, KVH, P = 64, 32, 8, 8192
    suf = bench_suffix_lengths()
    assert int(suf.sum()) == 33787  # the bench's workload (config.workload names this count)
    q16, k16, v16, bt_pre, bt_suf, suf = make_inputs(B, H, KVH, P, suf, seed=11)
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    print("cascade benchmark workload: B=%d H=%d KVH=%d prefix=%d suffix tokens=%d" % (B, H, KVH, P, suf.sum()),
          flush=True)
    outs = []
    for _ in range(10):
        outs.append(run_cascade(q, k, v, bt_pre, P, bt_suf, suf))
    torch.cuda.synchronize()
    out0, lse0 = outs[0]
    for i, (o, l) in enumerate(outs[1:], 1):
        assert torch.equal(o.view(torch.int16), out0.view(torch.int16)), "call %d differs from call 0 (O)" % i
        assert torch.equal(l.view(torch.int32), lse0.view(torch.int32)), "call %d differs from call 0 (LSE)" % i
    got = bf16_to_np(out0)
    lse = lse0.cpu().numpy().reshape(B, H).astype(np.float64)
    assert np.isfinite(got).all() and np.isfinite(lse).all()

    qf, kf, vf = bits_to_f32(q16), bits_to_f32(k16), bits_to_f32(v16)
    Od, Ld = dense_cascade(qf, kf, vf, bt_pre, P, bt_suf, suf)
    check_rows("cascade bench workload", got, lse, Od, Ld, "fp64 dense")
    Om, Lm = oracle_cascade(qf, kf, vf, bt_pre, P, bt_suf, suf)
    check_rows("cascade bench workload", got, lse, Om, Lm, "oracle composition")


def test_suffix_benchmark_workload_bit_stable():
    """The suffix op at the benchmark's suffix shape: ten calls bit-identical and
    every row equal to the oracle's fp32-P suffix attention."""
    B, H, KVH = 64, 32, 8
    suf = bench_suffix_lengths()
    q16, k16, v16, _, bt_suf, suf = make_inputs(B, H, KVH, 0, suf, seed=12)
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    bt = torch.from_numpy(bt_suf).to(DEV)
    sl = torch.from_numpy(suf).to(DEV)
    outs = [torch.ops.npu.suffix_decode(q, k, v, bt, sl) for _ in range(10)]
    torch.cuda.synchronize()
    for i, (o, l) in enumerate(outs[1:], 1):
        assert torch.equal(o.view(torch.int16), outs[0][0].view(torch.int16)), "call %d differs (O)" % i
        assert torch.equal(l.view(torch.int32), outs[0][1].view(torch.int32)), "call %d differs (LSE)" % i
    qf, kf, vf = bits_to_f32(q16), bits_to_f32(k16), bits_to_f32(v16)
    O_ref, L_ref = A.stage1(qf, kf, vf, bt_suf, np.ones(B, dtype=np.int64), suf, quantize_p=False)
    check_rows("suffix bench workload", bf16_to_np(outs[0][0]), outs[0][1].cpu().numpy().reshape(B, H), O_ref,
               L_ref, "oracle")


def fused_chunk_segments(suf, kv_groups, split=208):
    """Most sequences any fused chunk holds (host restatement of the kernel's chunk
    map: 32-token windows, 256 / kv_groups chunk pairs per kv head group, the first
    chunk of a pair taking split / 256 of the pair's windows)."""
    wins = [(int(s) + 31) // 32 for s in suf]
    cw = np.concatenate([[0], np.cumsum(wins)])
    W = int(cw[-1])
    pairs = 256 // kv_groups

    def lo(c):
        j = c >> 1
        a = j * W // pairs
        return a if c % 2 == 0 else a + (((j + 1) * W // pairs - a) * split >> 8)
    most = 0
    for c in range(2 * pairs):
        c0, c1 = lo(c), lo(c + 1)
        segs = sum(1 for b in range(len(suf)) if cw[b + 1] > cw[b] and cw[b] < c1 and cw[b + 1] > c0)
        most = max(most, segs)
    return most


MULTI_PHASE = [(768, 1024, 40, 5), (1024, 512, 20, 6)]


@pytest.mark.parametrize("B,P,maxlen,seed", MULTI_PHASE, ids=["b768_suf0-40", "b1024_suf0-20"])
def test_fused_chunks_spanning_table_phases(B, P, maxlen, seed):
    """H32 / KVH8 (4 query heads per kv head: the token-major streaming loop) with
    hundreds of short suffixes, some empty: fused chunks hold more than the 8
    sequences of one table phase, so the loop crosses phase boundaries (q-slot
    reset, the pipelined step's pending window, the drain). Every row against
    fp64 dense attention over prefix + suffix and the oracle's composition."""
    H, KVH = 32, 8
    rng = np.random.default_rng(seed)
    suf = rng.integers(1, maxlen + 1, size=B)
    suf[rng.random(B) < 0.1] = 0
    assert fused_chunk_segments(suf, KVH) > 8  # the premise: chunks span phases
    q16, k16, v16, bt_pre, bt_suf, suf = make_inputs(B, H, KVH, P, suf, seed)
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    print("multi-phase fused cascade: B=%d prefix=%d suffix max %d seed %d" % (B, P, maxlen, seed), flush=True)
    out, lse = run_cascade(q, k, v, bt_pre, P, bt_suf, suf)
    out2, lse2 = run_cascade(q, k, v, bt_pre, P, bt_suf, suf)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    got = bf16_to_np(out)
    L = lse.cpu().numpy().reshape(B, H).astype(np.float64)
    qf, kf, vf = bits_to_f32(q16), bits_to_f32(k16), bits_to_f32(v16)
    Od, Ld = dense_cascade(qf, kf, vf, bt_pre, P, bt_suf, suf)
    check_rows("fused multi-phase B=%d" % B, got, L, Od, Ld, "fp64 dense")
    Om, Lm = oracle_cascade(qf, kf, vf, bt_pre, P, bt_suf, suf)
    check_rows("fused multi-phase B=%d" % B, got, L, Om, Lm, "oracle composition")
