"""bfloat16 helpers on plain numpy (no ml_dtypes). Test infrastructure only.

``round_bf16`` restates the ``bf16()`` quantiser of
``ascend-kernel/csrc/ops/fa_fp32_stage1/test/fa_fp32_ref.py:25-27`` (ml_dtypes
RNE cast): float32 bits + 0x7FFF + lsb-of-upper-half, truncated to the upper 16
bits; NaN stays NaN. Pinned against torch's CPU float32 -> bfloat16 cast in
``tests/test_oracle_bf16.py``.
"""
import numpy as np


def bf16_bits(x):
    """float -> uint16 bfloat16 bit patterns (round to nearest, ties to even)."""
    x32 = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x32.view(np.uint32).astype(np.uint64)
    rne = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    out = (rne & np.uint64(0xFFFF)).astype(np.uint16)
    nan = np.isnan(x32)
    if nan.any():
        out = np.where(nan, ((u >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16), out)
    return out


def bits_to_f32(bits):
    """uint16 bfloat16 bit patterns -> float32 values (exact)."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x):
    """Round to the nearest bfloat16 value; returned as float32 (exact values)."""
    return bits_to_f32(bf16_bits(x))
