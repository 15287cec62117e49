"""GPU parity of lse_merge (torch op and C ABI) against the oracle and against the
reference kernel's reported error magnitudes on the same seeded inputs."""
import json
import os

import numpy as np
import pytest
import torch

from oracle.bf16 import round_bf16
from oracle.inputs import merge_inputs
from oracle.merge import merge_fp32, merge_fp64
from tests._util import MERGE_BOUNDARY, MERGE_MODES, MERGE_SHAPES, case_seed, merge_boundary, merge_metrics

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import cascade_amd  # noqa: F401
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def _report():
    path = os.path.join(os.path.dirname(__file__), "golden", "lse_merge", "lse_merge_precision_report.json")
    return {c["case"]: c for c in json.load(open(path))["cases"]}


def _run_case(mode, T, H, D, seed, boundary=None):
    o1_f32, out_code, padded, mere_tol, mare_tol, floor = MERGE_MODES[mode]
    o1, o2, l1c, l2c, l1, l2 = merge_inputs(T, H, D, o1_f32, padded, seed)
    if boundary:
        merge_boundary(boundary, o1, o2, l1, l2)
        if padded:
            l1c = l1.unsqueeze(-1).expand(T, H, 8).contiguous().reshape(T, H * 8)
            l2c = l2.unsqueeze(-1).expand(T, H, 8).contiguous().reshape(T, H * 8)
        else:
            l1c, l2c = l1, l2
    out = torch.ops.npu.lse_merge(o1.to(DEV), o2.to(DEV), l1c.to(DEV), l2c.to(DEV), out_code)
    torch.cuda.synchronize()
    ref, _ = merge_fp64(o1.double().numpy(), o2.double().numpy(), l1.double().numpy(), l2.double().numpy())
    bf16_out = out.dtype == torch.bfloat16
    got = out.float().cpu().numpy()
    refc = round_bf16(ref) if bf16_out else ref.astype(np.float32)
    return got, refc, (mere_tol, mare_tol, floor, 2e-2 if bf16_out else 1e-5), out.dtype


@pytest.mark.parametrize("mode", list(MERGE_MODES))
@pytest.mark.parametrize("shape", MERGE_SHAPES, ids=[s[0] for s in MERGE_SHAPES])
def test_reference_cases(mode, shape):
    cat, (T, H, D) = shape
    got, ref, (mere, mare, floor, abs_bound), dt = _run_case(mode, T, H, D, case_seed(f"{cat}/{mode}"))
    expect = torch.bfloat16 if mode in ("A_tier0", "C_hybrid_bf16", "D_tier0_pad") else torch.float32
    assert dt == expect
    m = merge_metrics(got, ref, floor)
    assert m["MERE"] < mere and m["MARE"] < mare and m["MaxAbsErr"] < abs_bound, m
    rep = _report()[f"{mode}/{cat}/{T}x{H}x{D}"]
    slack = 2.0 ** -7 if abs_bound > 1e-3 else 5e-7
    assert m["MaxAbsErr"] <= rep["MaxAbsErr"] + slack, (m, rep["MaxAbsErr"])


@pytest.mark.parametrize("mode", ["A_tier0", "B_fp32out", "C_hybrid_bf16", "Bp_fp32out_pad"])
@pytest.mark.parametrize("bname", MERGE_BOUNDARY)
def test_boundary_cases(mode, bname):
    got, ref, (mere, mare, floor, abs_bound), _ = _run_case(mode, 64, 40, 128, case_seed(bname), bname)
    m = merge_metrics(got, ref, floor)
    assert m["MERE"] < mere and m["MARE"] < mare and m["MaxAbsErr"] < abs_bound, m


def test_matches_fp32_oracle_order():
    """fp32 out vs the fp32 restatement of the kernel's operation order: within 2 ulp."""
    o1, o2, _, _, l1, l2 = merge_inputs(64, 40, 128, True, False, 7)
    out = torch.ops.npu.lse_merge(o1.to(DEV), o2.to(DEV), l1.to(DEV), l2.to(DEV), 2).cpu().numpy()
    ref, _ = merge_fp32(o1.numpy(), o2.float().numpy(), l1.numpy(), l2.numpy())
    assert np.abs(out - ref).max() <= 4 * np.spacing(np.abs(ref).max())


def test_padded_equals_compact_bitwise():
    T, H, D = 64, 40, 128
    g = torch.Generator().manual_seed(0)
    o1 = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(DEV)
    o2 = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(DEV)
    l1 = torch.randn(T, H, generator=g).to(DEV)
    l2 = torch.randn(T, H, generator=g).to(DEV)
    l1p = l1.unsqueeze(-1).expand(T, H, 8).contiguous().reshape(T, H * 8)
    l2p = l2.unsqueeze(-1).expand(T, H, 8).contiguous().reshape(T, H * 8)
    a = torch.ops.npu.lse_merge(o1, o2, l1, l2, 2)
    b = torch.ops.npu.lse_merge(o1, o2, l1p, l2p, 2)
    assert torch.equal(a, b)


def test_neg_inf_and_empty_suffix():
    T, H, D = 33, 8, 128
    g = torch.Generator().manual_seed(1)
    o1 = torch.randn(T, H, D, generator=g)
    o2 = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    l1 = torch.randn(T, H, generator=g)
    l2 = torch.randn(T, H, generator=g)
    l2[::3] = -float("inf")           # empty suffix rows
    l1[5, :] = -float("inf")          # empty prefix rows
    l2[5, 0] = -float("inf")          # both empty
    o2[0] = float("nan")              # filler in an empty-suffix row must not leak
    out, lse = torch.ops.npu.lse_merge_with_lse(o1.to(DEV), o2.to(DEV), l1.to(DEV), l2.to(DEV), 2)
    out, lse = out.cpu(), lse.cpu()
    emp = torch.isinf(l2) & torch.isfinite(l1)
    assert torch.equal(out[emp], o1[emp]) and torch.equal(lse[emp], l1[emp])
    emp1 = torch.isinf(l1) & torch.isfinite(l2)
    assert torch.equal(out[emp1], o2.float()[emp1]) and torch.equal(lse[emp1], l2[emp1])
    assert torch.all(out[5, 0] == 0) and lse[5, 0] == -float("inf")
    assert torch.isfinite(out).all()


def test_config3_fp32_partials_with_merged_lse_through_abi():
    """[256,32,128] fp32 o1/o2 ~ N(0,1), lse ~ N(0, sd 2), 5% of
    the suffix LSEs -inf; bf16 out + fp32 merged LSE, called through the C ABI."""
    from cascade_amd import abi
    rng = np.random.default_rng(0)
    B, H, D = 256, 32, 128
    o1 = rng.standard_normal((B, H, D)).astype(np.float32)
    o2 = rng.standard_normal((B, H, D)).astype(np.float32)
    l1 = (rng.standard_normal((B, H)) * 2).astype(np.float32)
    l2 = (rng.standard_normal((B, H)) * 2).astype(np.float32)
    l2[rng.random((B, H)) < 0.05] = -np.inf
    t = [torch.from_numpy(x).to(DEV) for x in (o1, o2, l1, l2)]
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(B, H, dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    rc = abi.lib().ck_lse_merge(t[0].data_ptr(), abi.CK_DTYPE_F32, t[1].data_ptr(), abi.CK_DTYPE_F32,
                                t[2].data_ptr(), 1, t[3].data_ptr(), 1, out.data_ptr(), abi.CK_DTYPE_BF16,
                                lse.data_ptr(), B * H, D, stream)
    abi.check(rc)
    torch.cuda.synchronize()
    ref, lref = merge_fp64(o1, o2, l1, l2)
    got = out.float().cpu().numpy()
    # bf16 output: within half an ulp of the fp64 result plus fp32 arithmetic noise
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6)
    lg = lse.cpu().numpy()
    assert np.abs(lg - lref).max() <= 1e-4 * np.abs(lref).max()
    # torch-op path agrees bit for bit with the ABI path
    out2, lse2 = torch.ops.npu.lse_merge_with_lse(t[0], t[1], t[2], t[3], 1)
    assert torch.equal(out2, out) and torch.equal(lse2, lse)


def test_rejections():
    o1 = torch.randn(2, 4, 16, device=DEV).to(torch.bfloat16)
    l1 = torch.randn(2, 4, device=DEV)
    with pytest.raises(RuntimeError, match="lse_merge"):
        torch.ops.npu.lse_merge(o1, o1, l1, l1, 3)
    with pytest.raises(RuntimeError, match="o2 must be bf16"):
        torch.ops.npu.lse_merge(o1.float(), o1.float(), l1, l1)
    empty = torch.empty(0, 4, 16, device=DEV, dtype=torch.bfloat16)
    assert torch.ops.npu.lse_merge(empty, empty, l1[:0], l1[:0]).shape == (0, 4, 16)
