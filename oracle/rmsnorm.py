"""Residual add + RMSNorm statistics oracle (numpy, fp64). Test infrastructure only.

Restates ``cpu_ref`` of ``ascend-kernel/csrc/ops/add_rms_norm_stats/test/add_rms_norm_stats_ref.py:139-156``
(the reference's fp64 model of the op; the semantics are design.md:37-62):

    xo    = x1                       (mode 1: the input already is the rounded residual)
          = rd(x1 + x2)              (modes 0, 2)
    rstd  = 1 / sqrt(mean_k(xo^2) + eps)          fp64, returned as fp32
    x_out = xo                       (mode 0)
    y     = rd(rd(xo * rstd) * gamma + beta)      (mode 1; beta None = no bias)

``rd`` is the reference's ``.to(dtype)`` of an fp64 tensor. torch converts
double -> bfloat16 / float16 through float32 (two round-to-nearest-even steps;
pinned in tests/test_oracle_rmsnorm.py), so ``rd`` here is fp64 -> fp32 -> dtype.
"""
import numpy as np

from .bf16 import round_bf16

DTYPES = ("bf16", "fp16")


def rd(x, dtype):
    """fp64 values -> the nearest dtype values via fp32 (as torch's cast), as fp64."""
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(x32).astype(np.float64)
    if dtype == "fp16":
        return x32.astype(np.float16).astype(np.float64)
    raise ValueError(dtype)


def add_rms_norm_stats(x1, x2, gamma, beta, eps, mode, dtype):
    """x1/x2 [M, K], gamma/beta [K] hold dtype values (any float array type).

    Returns (x_out, rstd, y) as fp64 arrays (rstd [M] already rounded to fp32);
    outputs the mode does not produce are None.
    """
    x1 = np.asarray(x1, dtype=np.float64)
    if mode == 1:
        xo = x1
    else:
        xo = rd(x1 + np.asarray(x2, dtype=np.float64), dtype)
    rstd = 1.0 / np.sqrt((xo * xo).mean(axis=-1) + eps)
    x_out = xo if mode == 0 else None
    y = None
    if mode == 1:
        acc = rd(xo * rstd[:, None], dtype) * np.asarray(gamma, dtype=np.float64)[None, :]
        if beta is not None:
            acc = acc + np.asarray(beta, dtype=np.float64)[None, :]
        y = rd(acc, dtype)
    return x_out, rstd.astype(np.float32).astype(np.float64), y
