"""HIP-graph capture of the graph-mode entry points.

The reference's caller replays its decode step as a graph (ascend-kernel/README.md:239-245)
and requires the q_seqlen_value > 0 fast path of fa_fp32_stage1 to be capture safe
(no device-to-host copy, tiling a pure function of shapes; op_host/fa_fp32_stage1.cpp:36-78).
Each op below is captured once into a torch.cuda.CUDAGraph and replayed several
times: before every replay fresh inputs are copied into the captured buffers, eager
work and a synchronisation run between replays, and every replay must equal the
eager result on the same inputs bit for bit (the kernels are deterministic: no
atomics, fixed launch shapes).
"""
import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits
from tests._util import torch_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("no_wait_giveups")]
DEV = "cuda:0"
REPLAYS = 3


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import cascade_amd  # noqa: F401
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def _bf16(rng, shape, scale=1.0):
    return torch_bf16(bf16_bits(rng.standard_normal(shape).astype(np.float32) * scale), DEV)


def _replay_check(make_inputs, op):
    """make_inputs(seed) -> list of tensors; op(*tensors) -> tuple of tensors."""
    static = make_inputs(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            op(*static)  # warm-up on the capture stream (one-time attribute setup)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = op(*static)
    outs = outs if isinstance(outs, (tuple, list)) else (outs,)
    filler = torch.randn(1024, 1024, device=DEV)
    for r in range(1, REPLAYS + 1):
        fresh = make_inputs(r)
        for s, f in zip(static, fresh):
            s.copy_(f)
        g.replay()
        filler = filler @ filler.t() * 1e-3  # unrelated eager work between replays
        torch.cuda.synchronize()
        ref = op(*fresh)
        ref = ref if isinstance(ref, (tuple, list)) else (ref,)
        torch.cuda.synchronize()
        for o, e in zip(outs, ref):
            if o is None:
                continue
            assert o.shape == e.shape and o.dtype == e.dtype
            assert torch.equal(o, e), "replay %d differs from eager" % r
    del g


def test_graph_stage1_fast_path():
    B, H, KVH, P = 16, 32, 8, 1536
    npages = P // 128

    def make(seed):
        rng = np.random.default_rng(seed)
        q = _bf16(rng, (B, H, 128))
        k = _bf16(rng, (2 * npages, 128, KVH, 128))
        v = _bf16(rng, (2 * npages, 128, KVH, 128))
        bt = torch.from_numpy(rng.permutation(2 * npages)[:npages].astype(np.int32)[None]).to(DEV)
        ql = torch.tensor([B], dtype=torch.int64, device=DEV)
        kl = torch.tensor([P - 37 * seed], dtype=torch.int64, device=DEV)
        return [q, k, v, bt, ql, kl]

    _replay_check(make, lambda q, k, v, bt, ql, kl: torch.ops.npu.fa_fp32_stage1(q, k, v, bt, ql, kl, B))


def test_graph_suffix_decode():
    B, H, KVH, cols = 12, 32, 8, 6
    nblocks = B * cols

    def make(seed):
        rng = np.random.default_rng(10 + seed)
        q = _bf16(rng, (B, H, 128))
        k = _bf16(rng, (nblocks, 128, KVH, 128))
        v = _bf16(rng, (nblocks, 128, KVH, 128))
        bt = torch.from_numpy(rng.permutation(nblocks).astype(np.int32).reshape(B, cols)).to(DEV)
        kl = torch.from_numpy(rng.integers(0, cols * 128 + 1, size=B).astype(np.int64)).to(DEV)
        return [q, k, v, bt, kl]

    _replay_check(make, lambda q, k, v, bt, kl: torch.ops.npu.suffix_decode(q, k, v, bt, kl))


def test_graph_lse_merge():
    rows, D = 512, 128

    def make(seed):
        rng = np.random.default_rng(20 + seed)
        o1 = torch.from_numpy(rng.standard_normal((rows, D)).astype(np.float32)).to(DEV)
        o2 = _bf16(rng, (rows, D))
        l1 = torch.from_numpy((rng.standard_normal(rows) * 2).astype(np.float32)).to(DEV)
        l2np = (rng.standard_normal(rows) * 2).astype(np.float32)
        l2np[rng.random(rows) < 0.05] = -np.inf
        l2 = torch.from_numpy(l2np).to(DEV)
        return [o1, o2, l1, l2]

    _replay_check(make, lambda o1, o2, l1, l2: torch.ops.npu.lse_merge_with_lse(o1, o2, l1, l2, 1))


def test_graph_cascade_decode():
    B, H, KVH, P, cols = 16, 32, 8, 1024, 5
    npre = P // 128
    nblocks = npre + B * cols

    def make(seed):
        rng = np.random.default_rng(30 + seed)
        q = _bf16(rng, (B, H, 128))
        k = _bf16(rng, (nblocks, 128, KVH, 128))
        v = _bf16(rng, (nblocks, 128, KVH, 128))
        perm = rng.permutation(nblocks).astype(np.int32)
        btp = torch.from_numpy(perm[:npre][None].copy()).to(DEV)
        bts = torch.from_numpy(perm[npre:].reshape(B, cols).copy()).to(DEV)
        pl = torch.tensor([P], dtype=torch.int64, device=DEV)
        sl = torch.from_numpy(rng.integers(0, cols * 128 + 1, size=B).astype(np.int64)).to(DEV)
        return [q, k, v, btp, pl, bts, sl]

    _replay_check(make, lambda q, k, v, btp, pl, bts, sl:
                  torch.ops.npu.cascade_decode(q, k, v, btp, pl, k, v, bts, sl))


def test_graph_swiglu_gemm():
    M, K, I = 256, 512, 384

    def make(seed):
        rng = np.random.default_rng(40 + seed)
        a = _bf16(rng, (M, K))
        b = _bf16(rng, (2 * I, K), 0.02)
        return [a, b]

    # mode 1 writes only d (the fused epilogue never stores C); mode 2 writes C into the workspace
    _replay_check(make, lambda a, b: torch.ops.npu.f3_gateup_epilogue(a, b, None, None, 1)[0])
    _replay_check(make, lambda a, b: torch.ops.npu.f3_gateup_epilogue(a, b, None, None, 2)[1])


def test_graph_add_rms_norm_stats():
    M, K = 96, 1024

    def make(seed):
        rng = np.random.default_rng(50 + seed)
        return [_bf16(rng, (M, K), 0.5), _bf16(rng, (M, K), 0.5), _bf16(rng, (K,), 0.1)]

    for mode in (0, 1, 2):
        _replay_check(make, lambda x1, x2, gm: torch.ops.npu.add_rms_norm_stats(x1, x2, gm, None, 1e-6, mode))
