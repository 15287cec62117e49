"""GPU checks of the two benchmark-only probes behind the bench line's measured
denominators (ck_bw_probe, ck_mfma_probe): they move / compute exactly what they
claim, so the rates derived from them are rates of that work."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def L():
    import cascade_amd  # noqa: F401
    from cascade_amd import abi
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")
    return abi


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# sizes that are not a multiple of the probe's grid stride (2048 x 256 lanes of 16 B),
# plus the smallest legal size
@pytest.mark.parametrize("nbytes", [16, 8 * 2**20 + 48, 40 * 2**20 + 16 * 1234])
def test_bw_probe_copy_is_exact(L, nbytes):
    g = torch.Generator(device=DEV).manual_seed(nbytes % 1000)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=DEV, generator=g)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=DEV)  # 64 guard bytes past the copy
    L.check(L.lib().ck_bw_probe(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), nbytes, 1,
                                None, 0, _stream()), "ck_bw_probe copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].count_nonzero()) == 0


@pytest.mark.parametrize("nbytes", [16, 8 * 2**20 + 48, 40 * 2**20 + 16 * 1234])
def test_bw_probe_read_touches_every_word_once(L, nbytes):
    """Each lane XOR-folds the 32-bit words of its 16-byte loads into its sink word,
    so the XOR of all sink words is the XOR of all words of the source exactly when
    every 16-byte element was loaded an odd number of times (once, by the grid)."""
    g = torch.Generator(device=DEV).manual_seed(7 + nbytes % 1000)
    src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=DEV, generator=g)
    sink = torch.full((L.PROBE_SINK_BYTES // 4,), -1, dtype=torch.int32, device=DEV)
    L.check(L.lib().ck_bw_probe(ctypes.c_void_p(src.data_ptr()), None, nbytes, 0, ctypes.c_void_p(sink.data_ptr()),
                                L.PROBE_SINK_BYTES, _stream()), "ck_bw_probe read")
    torch.cuda.synchronize()
    s = sink.cpu().numpy().view(np.uint32)
    want = np.bitwise_xor.reduce(src.cpu().numpy().view(np.uint32))
    assert int(np.bitwise_xor.reduce(s)) == int(want)
    # lanes past the data (small sizes) still write their (empty) fold: 0
    if nbytes == 16:
        assert int(s[0]) == int(want) and not s[1:].any()


def _bf16(x):
    return torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).to(torch.float64).numpy()


@pytest.mark.parametrize("iters", [1, 37])
def test_mfma_probe_runs_every_mfma(L, iters):
    """Every wave runs 8 accumulators x 2 iters MFMAs of the same 32x32x16 product C
    (A[i][k] = bf16(1 + 1e-3 lane + 1e-2 e) on the lane holding row i, B likewise
    with minus signs), so each wave's 64 sink values sum to 16 iters sum(C), and
    sum(C) = sum_k (sum_i A[i][k]) (sum_j B[k][j]) whatever the fragment layout."""
    sink = torch.zeros(L.PROBE_SINK_BYTES // 4, dtype=torch.float32, device=DEV)
    flops = ctypes.c_double(0.0)
    L.check(L.lib().ck_mfma_probe(iters, ctypes.c_void_p(sink.data_ptr()), L.PROBE_SINK_BYTES, ctypes.byref(flops),
                                  _stream()), "ck_mfma_probe")
    torch.cuda.synchronize()
    waves = 512 * 4
    assert flops.value == waves * iters * 16 * (2.0 * 32 * 32 * 16)
    a = np.zeros((32, 16))
    b = np.zeros((16, 32))
    for lane in range(64):
        row, kb = lane % 32, lane // 32
        for e in range(8):
            a[row, 8 * kb + e] = _bf16(1.0 + 1e-3 * lane + e * 1e-2)
            b[8 * kb + e, row] = _bf16(1.0 - 1e-3 * lane - e * 1e-2)
    want = 16 * iters * float((a.sum(axis=0) * b.sum(axis=1)).sum())
    per_wave = sink[: waves * 64].double().reshape(waves, 64).sum(dim=1).cpu().numpy()
    np.testing.assert_allclose(per_wave, want, rtol=1e-5)
    assert not sink[waves * 64:].any()  # the grid writes only its own lanes
