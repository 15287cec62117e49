"""GPU parity of ck_cascade_decode_noalloc (the cascade with its workspace in the
library's device scratch array) against ck_cascade_decode with a caller
workspace, on two calls in a row, the second one smaller: the outputs must be
bit-identical (the same kernels on the same inputs; only the workspace differs),
including after the first call has left its partials in the shared array."""
import ctypes

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits
from tests._util import torch_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("no_wait_giveups")]
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import cascade_amd  # noqa: F401
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def _case(B, H, KVH, P, seed):
    rng = np.random.default_rng(seed)
    suf = np.clip(rng.geometric(1 / 300, size=B), 1, 2000).astype(np.int64)
    suf[::5] = 0  # some empty suffixes
    nsb = [(int(s) + 127) // 128 for s in suf]
    nblocks = P // 128 + sum(nsb)
    k = bf16_bits(rng.standard_normal((nblocks, 128, KVH, 128)))
    v = bf16_bits(rng.standard_normal((nblocks, 128, KVH, 128)))
    q = bf16_bits(rng.standard_normal((B, H, 128)))
    perm = rng.permutation(nblocks).astype(np.int32)
    bt_pre = perm[:P // 128][None, :].copy()
    bt_suf = np.zeros((B, max(max(nsb), 1)), dtype=np.int32)
    off = P // 128
    for b in range(B):
        bt_suf[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    t = dict(q=torch_bf16(q, DEV), k=torch_bf16(k, DEV), v=torch_bf16(v, DEV),
             btp=torch.from_numpy(bt_pre).to(DEV), bts=torch.from_numpy(bt_suf).to(DEV),
             plen=torch.tensor([P], dtype=torch.int64, device=DEV), sl=torch.from_numpy(suf).to(DEV))
    return t


def _args(t, B, H, KVH, out, lse):
    pcap, scap = t["btp"].shape[1] * 128, t["bts"].shape[1] * 128
    nb = t["k"].shape[0]
    return (t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), t["btp"].data_ptr(), t["btp"].shape[1],
            t["plen"].data_ptr(), nb, t["k"].data_ptr(), t["v"].data_ptr(), t["bts"].data_ptr(), t["bts"].shape[1],
            t["sl"].data_ptr(), nb, 0, B, H, KVH, 128, 128, float(np.float32(1 / np.sqrt(128.0))), pcap, scap,
            out.data_ptr(), lse.data_ptr())


def test_noalloc_matches_workspace_entry_two_calls():
    from cascade_amd import abi
    L = abi.lib()
    stream = torch.cuda.current_stream().cuda_stream
    # second call smaller than the first: it must not see the first call's partials
    for (B, H, KVH, P, seed) in [(48, 32, 8, 4096, 1), (7, 16, 4, 640, 2)]:
        print("noalloc case B=%d H=%d KVH=%d P=%d" % (B, H, KVH, P), flush=True)
        t = _case(B, H, KVH, P, seed)
        pcap, scap = t["btp"].shape[1] * 128, t["bts"].shape[1] * 128
        wsb = abi.cascade_plan(B, H, KVH, 128, pcap, scap)
        assert 0 < wsb <= abi.CASCADE_NOALLOC_SCRATCH_BYTES
        ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
        out1 = torch.empty(B, H, 128, dtype=torch.bfloat16, device=DEV)
        lse1 = torch.empty(B * H, dtype=torch.float32, device=DEV)
        out2 = torch.full_like(out1, float("nan"))
        lse2 = torch.full_like(lse1, float("nan"))
        a1 = _args(t, B, H, KVH, out1, lse1)
        abi.check(L.ck_cascade_decode(*a1, ws.data_ptr(), wsb, stream), "ck_cascade_decode")
        abi.check(L.ck_cascade_decode_noalloc(*_args(t, B, H, KVH, out2, lse2), stream),
                  "ck_cascade_decode_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out1, out2)
        assert torch.equal(lse1.view(torch.int32), lse2.view(torch.int32))


def test_noalloc_under_graph_capture():
    """The callers it is for capture it: one eager call on the capture stream (the
    per-device set-up happens there), then the call captured into a HIP graph and
    replayed twice, each time after fresh q/K/V values and rotated suffix lengths
    were copied into the captured buffers, with unrelated eager work between the
    replays. Each replay equals ck_cascade_decode with a caller workspace on the
    same inputs, bit for bit."""
    from cascade_amd import abi
    L = abi.lib()
    B, H, KVH, P = 24, 32, 8, 2048
    t = _case(B, H, KVH, P, 3)
    out = torch.empty(B, H, 128, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(B * H, dtype=torch.float32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        abi.check(L.ck_cascade_decode_noalloc(*_args(t, B, H, KVH, out, lse), side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        abi.check(L.ck_cascade_decode_noalloc(*_args(t, B, H, KVH, out, lse),
                                              torch.cuda.current_stream().cuda_stream))
    pcap, scap = t["btp"].shape[1] * 128, t["bts"].shape[1] * 128
    wsb = abi.cascade_plan(B, H, KVH, 128, pcap, scap)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(7)
    filler = torch.randn(512, 512, device=DEV)
    for r in (1, 2):
        print("noalloc graph replay %d" % r, flush=True)
        for name in ("q", "k", "v"):
            t[name].copy_(torch.randn(t[name].shape, generator=gen, device=DEV).to(torch.bfloat16))
        t["sl"].copy_(torch.roll(t["sl"], r))  # lengths stay within the captured caps
        g.replay()
        filler = filler @ filler.t() * 1e-3
        torch.cuda.synchronize()
        ref_out = torch.full_like(out, float("nan"))
        ref_lse = torch.full_like(lse, float("nan"))
        abi.check(L.ck_cascade_decode(*_args(t, B, H, KVH, ref_out, ref_lse), ws.data_ptr(), wsb,
                                      torch.cuda.current_stream().cuda_stream), "ck_cascade_decode")
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), "replay %d (O)" % r
        assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32)), "replay %d (LSE)" % r
    del g


def test_noalloc_refuses_shapes_beyond_its_scratch():
    from cascade_amd import abi
    L = abi.lib()
    B, H, KVH = 16384, 64, 8  # the plan's whole-sequence scratch alone exceeds 32 MiB
    assert abi.cascade_plan(B, H, KVH, 128, 128, 128) > abi.CASCADE_NOALLOC_SCRATCH_BYTES
    p = ctypes.c_void_p(256)  # never dereferenced: the call is refused first
    rc = L.ck_cascade_decode_noalloc(p, p, p, p, 1, p, 1, p, p, p, 1, p, 1, 0, B, H, KVH, 128, 128, 0.088, 128,
                                     128, p, p, None)
    assert rc == abi.CK_E_SCRATCH_LIMIT
