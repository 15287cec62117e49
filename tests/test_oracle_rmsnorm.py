"""Pins the add_rms_norm_stats oracle (oracle/rmsnorm.py).

* The cast: torch converts float64 -> bfloat16 / float16 through float32 (two
  RNE steps), which is what the reference's fp64 model (add_rms_norm_stats_ref.py:139-156)
  relies on and what oracle.rmsnorm.rd restates.
* Golden points: the element dumps the reference recorded in its golden self-check
  (f2_golden_selfcheck.json, via tests/golden/add_rms_norm_stats/make_golden.py).
  The inputs are re-created from each case's seed with the reference's generator
  (add_rms_norm_stats_cases.py:33-43). The dumped elements are the reference's own
  near-tie elements of y, so they are maximally sensitive: the oracle's rstd must
  agree with the recorded CANN rstd to 1e-6, and y with the recorded fp64-model
  value up to one flip of each of its two roundings; all but one point match
  exactly (the recorded rstd itself differs from CANN's by up to 5e-7 there).
* Closed forms: a constant row, idempotence of the rounding, mode consistency, and
  the residual output against torch's own bf16/fp16 addition.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle.rmsnorm import add_rms_norm_stats, rd

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "add_rms_norm_stats", "golden_selfcheck_points.json")
TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def make_inputs(m, k, dtype, seed, has_beta):
    """The reference's input generator (add_rms_norm_stats_cases.py:33-43), on the CPU."""
    dt = TORCH_DT[dtype]
    g = torch.Generator(device="cpu").manual_seed(seed)
    x1 = (torch.randn(m, k, generator=g, dtype=torch.float32) * 0.5).to(dt)
    x2 = (torch.randn(m, k, generator=g, dtype=torch.float32) * 0.5).to(dt)
    gamma = (1.0 + torch.randn(k, generator=g, dtype=torch.float32) * 0.1).to(dt)
    beta = (torch.randn(k, generator=g, dtype=torch.float32) * 0.05).to(dt) if has_beta else None
    return x1, x2, gamma, beta


def ulp(x, dtype):
    """Spacing of the dtype at |x| (normal range)."""
    mant = 7 if dtype == "bf16" else 10
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - mant)


def test_torch_double_cast_goes_through_float32():
    d = torch.tensor([1.0 + 2 ** -8 + 2 ** -30, 1.0 + 2 ** -11 + 2 ** -30], dtype=torch.float64)
    # correctly rounded these would be 1 + 2^-7 and 1 + 2^-10; through fp32 both become ties -> even
    assert d[:1].to(torch.bfloat16).double().item() == 1.0
    assert d[1:].to(torch.float16).double().item() == 1.0
    assert rd(d[:1].numpy(), "bf16")[0] == 1.0
    assert rd(d[1:].numpy(), "fp16")[0] == 1.0
    vals = np.random.default_rng(0).standard_normal(4096) * 3
    for dt, tdt in TORCH_DT.items():
        assert np.array_equal(rd(vals, dt), torch.from_numpy(vals).to(tdt).double().numpy())


def test_golden_selfcheck_points():
    data = json.load(open(GOLDEN))
    for case in data["cases"]:
        dtype = "bf16" if case["dtype"] == "bfloat16" else "fp16"
        x1, _, gamma, _ = make_inputs(case["m"], case["k"], dtype, case["seed"], has_beta=False)
        _, rstd, y = add_rms_norm_stats(x1.double().numpy(), None, gamma.double().numpy(), None, data["eps"], 1,
                                        dtype)
        exact = 0
        for e in case["elements"]:
            assert float(gamma[e["col"]]) == e["gamma"], "input generator does not reproduce the reference's"
            assert abs(rstd[e["row"]] / e["rstd_cann"] - 1.0) <= 1e-6
            got = y[e["row"], e["col"]]
            # at most one flip of each of the two roundings: rd(x * rstd) by one ulp
            # (times gamma), and the final rd() by one ulp
            g = abs(e["gamma"])
            bound = ulp(e["ref"] / g, dtype) * g + ulp(e["ref"], dtype)
            assert abs(got - e["ref"]) <= bound, (e, got)
            exact += got == e["ref"]
        assert exact >= len(case["elements"]) - 1, (case["case"], exact)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_closed_forms(dtype):
    k = 256
    c = np.array([0.5, 1.25, -3.0, 7.5])
    x1 = np.repeat(c[:, None], k, axis=1)
    _, rstd, _ = add_rms_norm_stats(x1, np.zeros_like(x1), None, None, 1e-6, 2, dtype)
    assert np.array_equal(rstd, (1.0 / np.sqrt(c * c + 1e-6)).astype(np.float32).astype(np.float64))
    x1t, x2t, gamma, beta = make_inputs(33, 512, dtype, 5, has_beta=True)
    x1n, x2n = x1t.double().numpy(), x2t.double().numpy()
    xo, r0, _ = add_rms_norm_stats(x1n, x2n, None, None, 1e-6, 0, dtype)
    # the residual output equals torch's own addition in float32 rounded to the dtype
    assert np.array_equal(xo, (x1t.float() + x2t.float()).to(TORCH_DT[dtype]).double().numpy())
    _, r2, _ = add_rms_norm_stats(x1n, x2n, None, None, 1e-6, 2, dtype)
    _, r1, y = add_rms_norm_stats(xo, None, gamma.double().numpy(), beta.double().numpy(), 1e-6, 1, dtype)
    assert np.array_equal(r0, r2) and np.array_equal(r0, r1)
    # gamma = 1, beta = 0: y is the rounded normalised residual and rounding is idempotent
    _, _, y1 = add_rms_norm_stats(xo, None, np.ones(512), None, 1e-6, 1, dtype)
    assert np.array_equal(y1, rd(xo * (1.0 / np.sqrt((xo * xo).mean(-1) + 1e-6))[:, None], dtype))
    assert np.array_equal(rd(y, dtype), y)
    # a planted mistake: the statistics of the unrounded sum differ from those of x_out
    s = x1n + x2n
    wrong = (1.0 / np.sqrt((s * s).mean(-1) + 1e-6)).astype(np.float32)
    assert not np.array_equal(wrong, r0.astype(np.float32))
