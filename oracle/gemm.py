"""gate_up GEMM + epilogue oracle (numpy). Test infrastructure only.

Restates ``ascend-kernel/csrc/ops/f3_floor``:
* weight layout: b is [2I, K] row-major (nn.Linear), gate rows 0..I-1 and up rows
  I..2I-1; C = a b^T with fp32 accumulation stored as bf16 RNE
  (``op_kernel/kernel_f3_floor.cpp:150-199``; ``design.md:98`` states C is bitwise
  ``F.linear``);
* epilogue windows: mode 0/5 D = C[:, :I], mode 4 D = C[:, I:]
  (``kernel_f3_floor.cpp:214-308``, ``design.md:94-103``);
* mode 1 SwiGLU: the reference leaves it as a hook (``design.md:107-109`` gives the
  chain cast-fp32, -x, exp, +1, div, *up, RNE). Here D = bf16(silu(g) * u) with g,u the
  fp32-accumulated products (no bf16 rounding of g,u: the fused epilogue reads the
  accumulators), silu(x) = x / (1 + exp(-x)) (``catlass/epilogue/tile/tile_elemwise_silu.hpp:34-46``).
Accumulation here is fp64 (exact for these sizes up to rounding), then rounded.
"""
import numpy as np

from .bf16 import round_bf16


def accumulate(a, b):
    """fp64 a @ b^T. a [M,K], b [N,K] (float arrays holding bf16 values)."""
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64).T


def gemm_c(a, b):
    """C = bf16_RNE(a b^T) [M, 2I] as float32 values."""
    return round_bf16(accumulate(a, b))


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def swiglu(a, b):
    """Mode-1 D = bf16_RNE(silu(gate) * up) [M, I] as float32 values; also returns the
    unrounded fp64 product for tolerance checks."""
    acc = accumulate(a, b)
    n_half = acc.shape[1] // 2
    exact = silu(acc[:, :n_half]) * acc[:, n_half:]
    return round_bf16(exact), exact


def epilogue(a, b, mode):
    """D for the window modes (0, 4, 5) and mode 1; None for modes that write no D."""
    c = gemm_c(a, b)
    n_half = c.shape[1] // 2
    if mode in (0, 5):
        return c[:, :n_half]
    if mode == 4:
        return c[:, n_half:]
    if mode == 1:
        return swiglu(a, b)[0]
    return None
