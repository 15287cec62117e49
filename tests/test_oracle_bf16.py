"""Pins oracle.bf16 against torch's CPU float32 -> bfloat16 cast (RNE)."""
import numpy as np
import torch

from oracle.bf16 import bf16_bits, bits_to_f32, round_bf16


def _torch_bits(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_random_values_match_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000), rng.standard_normal(10000) * 1e30,
                        rng.standard_normal(10000) * 1e-38]).astype(np.float32)
    assert np.array_equal(bf16_bits(x), _torch_bits(x))


def test_ties_round_to_even():
    # exact midpoints between bf16 neighbours: 1 + 2^-8 (tie -> even 1.0), 1 + 3*2^-8 (tie -> up)
    x = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 2 ** -130 * 1.5], dtype=np.float32)
    assert np.array_equal(bf16_bits(x), _torch_bits(x))
    assert round_bf16(x)[0] == 1.0 and round_bf16(x)[1] == 1 + 4 * 2 ** -8


def test_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, np.float32(np.finfo(np.float32).max)], dtype=np.float32)
    assert np.array_equal(bf16_bits(x), _torch_bits(x))
    nan = round_bf16(np.array([np.nan], dtype=np.float32))
    assert np.isnan(nan[0])


def test_roundtrip_exact():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = bits_to_f32(bits)
    finite = np.isfinite(f)
    assert np.array_equal(bf16_bits(f[finite]), bits[finite])


def test_truncation_is_detected():
    """Planted mistake: truncating instead of rounding must disagree with torch."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal(1000).astype(np.float32)
    trunc = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert not np.array_equal(trunc, _torch_bits(x))
