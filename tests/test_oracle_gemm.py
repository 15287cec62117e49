"""Pins oracle.gemm against torch CPU F.linear / F.silu and the epilogue-window
definitions of the f3 ladder."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle.bf16 import round_bf16
from oracle.gemm import epilogue, gemm_c, silu, swiglu


def _inputs(M, K, I, seed=0):
    rng = np.random.default_rng(seed)
    a = round_bf16(rng.standard_normal((M, K)))
    b = round_bf16(rng.standard_normal((2 * I, K)) * 0.02)
    return a, b


def test_c_matches_torch_linear():
    a, b = _inputs(33, 256, 128)
    c = gemm_c(a, b)
    t = F.linear(torch.from_numpy(a).double(), torch.from_numpy(b).double()).float().to(torch.bfloat16).float().numpy()
    # fp64 vs fp64 accumulation order: identical after bf16 rounding except at exact ties
    assert (c != t).mean() < 1e-3
    assert np.abs(c - t).max() <= 2.0 ** -7 * np.abs(t).max()


def test_silu_closed_forms():
    x = np.array([0.0, 50.0, -50.0, 1.0])
    s = silu(x)
    assert s[0] == 0 and abs(s[1] - 50) < 1e-15 and abs(s[2]) < 1e-19
    assert abs(s[3] - 1 / (1 + np.exp(-1))) < 1e-15
    y = np.random.default_rng(0).standard_normal(1000) * 4
    assert np.abs(silu(y) - F.silu(torch.from_numpy(y)).numpy()).max() < 1e-14


def test_swiglu_matches_torch():
    a, b = _inputs(17, 192, 128, seed=1)
    d, exact = swiglu(a, b)
    ta, tb = torch.from_numpy(a).double(), torch.from_numpy(b).double()
    g, u = F.linear(ta, tb[:128]), F.linear(ta, tb[128:])
    ref = (F.silu(g) * u).numpy()
    assert np.abs(exact - ref).max() < 1e-12
    assert np.array_equal(d, round_bf16(ref))


def test_window_modes_and_planted_swap():
    a, b = _inputs(16, 128, 256, seed=2)
    c = gemm_c(a, b)
    assert np.array_equal(epilogue(a, b, 0), c[:, :256])
    assert np.array_equal(epilogue(a, b, 5), c[:, :256])
    assert np.array_equal(epilogue(a, b, 4), c[:, 256:])
    assert epilogue(a, b, 2) is None
    # planted mistake: gate/up halves swapped is visible
    assert not np.array_equal(epilogue(a, b, 0), epilogue(a, b, 4))
    b_sw = np.concatenate([b[256:], b[:256]])
    assert not np.array_equal(swiglu(a, b)[0], swiglu(a, b_sw)[0])
