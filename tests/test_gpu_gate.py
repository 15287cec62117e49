"""GPU checks of the cascade-vs-full gate (cascade_amd/gate.py): the FULL form is
per-sequence decode over prefix + suffix pages and equals dense softmax attention
over the concatenated KV (the same criterion as BASELINE config 1 for the cascade);
both forms agree to the bf16-P bound; a real measurement yields a decision and the
dispatcher returns the chosen form's result."""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.bf16 import bf16_bits, bits_to_f32
from tests._util import bf16_to_np, torch_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("no_wait_giveups")]
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import cascade_amd  # noqa: F401
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def _case(B=8, H=32, KVH=8, P=1024, seed=3):
    rng = np.random.default_rng(seed)
    suf = rng.integers(0, 300, size=B)
    nsb = [max(1, (int(s) + 127) // 128) for s in suf]
    nblocks = P // 128 + sum(nsb)
    k = rng.standard_normal((nblocks, 128, KVH, 128)).astype(np.float32)
    v = rng.standard_normal((nblocks, 128, KVH, 128)).astype(np.float32)
    q = rng.standard_normal((B, H, 128)).astype(np.float32)
    perm = rng.permutation(nblocks).astype(np.int32)
    btp = perm[:P // 128][None].copy()
    bts = np.zeros((B, max(nsb)), dtype=np.int32)
    off = P // 128
    for b in range(B):
        bts[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    return bf16_bits(q), bf16_bits(k), bf16_bits(v), btp, bts, suf.astype(np.int64), P


def test_full_form_equals_dense_and_cascade():
    from cascade_amd import gate as G
    q16, k16, v16, btp, bts, suf, P = _case()
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    btp_t, bts_t = torch.from_numpy(btp).to(DEV), torch.from_numpy(bts).to(DEV)
    sl = torch.from_numpy(suf).to(DEV)
    of, lf = G.full_decode(q, k, v, btp_t, P, bts_t, sl)
    oc, lc = torch.ops.npu.cascade_decode(q, k, v, btp_t, torch.tensor([P], dtype=torch.int64, device=DEV),
                                          k, v, bts_t, sl)
    torch.cuda.synchronize()
    of, oc = bf16_to_np(of), bf16_to_np(oc)
    # dense softmax attention over prefix + own suffix, per sequence (fp64)
    full_bt = np.concatenate([np.repeat(btp, len(suf), 0), bts], axis=1)
    B, H = q16.shape[0], q16.shape[1]
    O_ref, L_ref = A.stage1(bits_to_f32(q16), bits_to_f32(k16), bits_to_f32(v16), full_bt, np.ones(B, np.int64),
                            suf + P, chunk=None, quantize_p=False)
    assert np.all(np.abs(of - O_ref) <= 2e-3 + 2.0 ** -8 * np.abs(O_ref))
    assert np.max(np.abs(lf.cpu().numpy().reshape(B, H) - L_ref) / np.maximum(np.abs(L_ref), 1.0)) <= 1e-4
    vmax = float(np.abs(bits_to_f32(v16)).max())
    assert np.max(np.abs(of - oc)) <= 2.0 ** -8 * vmax + 2.0 ** -7 * np.abs(O_ref).max()


def test_gate_measures_and_dispatches():
    from cascade_amd import gate as G
    g = G.CascadeGate(32, 8, suffix_len=256, shared_quantum=1024)
    choice = g.choose(8, 1024)
    d = g.decisions[(8, 1024)]
    assert choice in (G.CASCADE, G.FULL) and d["cascade_ms"] > 0 and d["full_ms"] > 0
    q16, k16, v16, btp, bts, suf, P = _case()
    q, k, v = (torch_bf16(x, DEV) for x in (q16, k16, v16))
    btp_t, bts_t = torch.from_numpy(btp).to(DEV), torch.from_numpy(bts).to(DEV)
    sl = torch.from_numpy(suf).to(DEV)
    out, lse = g.decode(q, k, v, btp_t, P, bts_t, sl)
    if choice == G.FULL:
        ref = G.full_decode(q, k, v, btp_t, P, bts_t, sl)
    else:
        ref = torch.ops.npu.cascade_decode(q, k, v, btp_t, torch.tensor([P], dtype=torch.int64, device=DEV),
                                           k, v, bts_t, sl)
    torch.cuda.synchronize()
    assert torch.equal(out, ref[0]) and torch.equal(lse, ref[1])
