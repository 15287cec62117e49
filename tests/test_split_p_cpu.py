"""The suffix kernels' P operand on the matrix cores: p (fp32, 0 <= p <= 2^8 after
the lazy running max) enters the bf16 MFMA as two terms, hi = p truncated to bf16
and lo = p - hi rounded to bf16 (csrc/suffix_decode.hip, the token-major step).
The kernel's contract is fp32-P precision: |hi + lo - p| <= 2^-16 p, so that the
value MFMA sums p * v to within fp32-level error of the unquantised oracle.

The bound follows from hi keeping p's top 8 significand bits (|p - hi| < 2^-7 p,
and p - hi is exact in fp32) and lo's RNE to 8 bits (error <= 2^-9 |p - hi|).
These checks pin it on random and adversarial values with the oracle's own RNE
(oracle/bf16.py, itself pinned against torch), and show the two plausible
mistakes miss it: hi alone (bf16 P) and a truncated lo term."""
import numpy as np

from oracle.bf16 import bits_to_f32, round_bf16


def _hi(p):
    return (p.astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def _split(p, lo_round=True):
    p = p.astype(np.float32)
    hi = _hi(p)
    d = (p - hi).astype(np.float32)  # exact: hi is p with its low 16 bits cleared
    lo = round_bf16(d) if lo_round else _hi(d)
    return hi, lo


def _p_values():
    rng = np.random.default_rng(0)
    p = np.concatenate([
        np.exp2(-rng.uniform(0, 60, 200000)),              # exp2(s - m) after the running max
        rng.uniform(0, 256, 100000),                        # up to 2^kTau above the max's reference
        np.float32(1.0) + np.arange(1, 4096, dtype=np.float32) * np.float32(2.0 ** -23),  # low bits set
        bits_to_f32(np.arange(0x3F80, 0x4380, dtype=np.uint16)),                            # exact bf16 values
        np.array([0.0, 2.0 ** -126, 255.99998, 256.0], dtype=np.float32),
    ]).astype(np.float32)
    return p


def test_difference_is_exact_in_fp32():
    p = _p_values()
    hi = _hi(p)
    d32 = (p - hi).astype(np.float32)
    np.testing.assert_array_equal(d32.astype(np.float64), p.astype(np.float64) - hi.astype(np.float64))


def test_hi_plus_lo_within_2_pow_minus_16():
    p = _p_values()
    hi, lo = _split(p)
    err = np.abs(hi.astype(np.float64) + lo.astype(np.float64) - p.astype(np.float64))
    assert np.all(err <= 2.0 ** -16 * p.astype(np.float64)), (err / np.maximum(p, 1e-300)).max()
    # exact bf16 values split into (p, 0)
    b = bits_to_f32(np.arange(0x3F80, 0x4380, dtype=np.uint16))
    hb, lb = _split(b)
    assert np.array_equal(hb, b) and not lb.any()


def test_plausible_mistakes_miss_the_bound():
    p = _p_values()
    pos = p > 0
    # bf16 P alone (hi only, or p rounded once): errors up to 2^-8 p
    hi, _ = _split(p)
    rel_hi = np.abs(hi.astype(np.float64) - p)[pos] / p[pos]
    rel_rne = np.abs(round_bf16(p).astype(np.float64) - p)[pos] / p[pos]
    assert rel_hi.max() > 2.0 ** -16 and rel_rne.max() > 2.0 ** -16
    # a truncated lo term (not rounded) doubles lo's error bound: 2^-16 is exceeded
    h2, l2 = _split(p, lo_round=False)
    rel_trunc = np.abs(h2.astype(np.float64) + l2.astype(np.float64) - p)[pos] / p[pos]
    assert rel_trunc.max() > 2.0 ** -16
