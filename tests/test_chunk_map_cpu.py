"""The window -> chunk arithmetic of the suffix kernels, the fix-up and the
cascade epilogue (`ChunkMap` in csrc/suffix_decode.hip), checked on the host.

The kernels take floor(x / d) as the truncated IEEE double quotient
(`div_nonneg`) for 0 <= x <= W P and 1 <= d < 2^31, where W < 2^31 windows (the
int32 prefix sums) and P <= 2^20 chunks (the ABI's limit). numpy's float64
division is the same correctly rounded IEEE operation, so these tests pin the
identity on random and adversarial operands (quotients just below an integer,
the largest operands), show that a single-precision quotient fails them, and
check the chunk map built on it: chunk c covers [lo(c), lo(c + 1)) and owner(p)
is the chunk whose range holds window p."""
import numpy as np
import pytest

X_MAX = (2 ** 31 - 1) * 2 ** 20  # W P at the limits


def _div(x, d, dtype=np.float64):
    return (x.astype(dtype) / d.astype(dtype)).astype(np.int64)


def _operands(rng, n):
    d = np.concatenate([rng.integers(1, 2 ** 31, n), rng.integers(1, 5000, n)])
    q = rng.integers(0, X_MAX // d + 1)
    x = np.concatenate([
        rng.integers(0, X_MAX + 1, 2 * n),                  # anywhere
        np.minimum(q * d + d - 1, X_MAX),                   # just below the next integer
        q * d,                                              # exact quotients
        np.maximum(q * d - 1, 0),
    ])
    return x, np.concatenate([d, d, d, d])


def test_double_quotient_is_the_integer_floor():
    rng = np.random.default_rng(0)
    for _ in range(8):
        x, d = _operands(rng, 250_000)
        assert ((x >= 0) & (x <= X_MAX)).all()
        np.testing.assert_array_equal(_div(x, d), x // d)
    # the extremes
    x = np.array([X_MAX, X_MAX - 1, 2 ** 31 - 2, 0, (2 ** 31 - 1) * (2 ** 20 - 1)], dtype=np.int64)
    d = np.array([2 ** 31 - 1, 2 ** 31 - 1, 2 ** 31 - 1, 1, 2 ** 20], dtype=np.int64)
    np.testing.assert_array_equal(_div(x, d), x // d)


def test_single_precision_quotient_would_fail():
    # the check has teeth: a float32 quotient misses the floor on these operands
    rng = np.random.default_rng(1)
    x, d = _operands(rng, 50_000)
    assert (_div(x, d, np.float32) != x // d).any()


def _lo(c, W, P, split):
    if split == 0:
        return _div(c * W, np.full_like(c, P))
    h, j = P // 2, c // 2
    a = _div(j * W, np.full_like(j, h))
    b = _div((j + 1) * W, np.full_like(j, h))
    return np.where(c % 2 == 0, a, a + (((b - a) * split) >> 8))


def _owner(p, W, P, split):
    if split == 0:
        return _div((p + 1) * P - 1, np.full_like(p, W))
    j = _div((p + 1) * (P // 2) - 1, np.full_like(p, W))
    return 2 * j + (p >= _lo(2 * j + 1, W, P, split))


@pytest.mark.parametrize("W,P,split", [
    (1, 1, 0), (7, 512, 0), (1088, 64, 0), (1088, 64, 192), (5, 64, 192), (33787, 512, 0),
    (2 ** 31 - 1, 2 ** 20, 0), (2 ** 31 - 1, 512, 192), (123457, 1000, 128), (2 ** 30 + 3, 2 ** 20, 255),
])
def test_chunk_map_ranges_and_owner(W, P, split):
    c = np.arange(P + 1, dtype=np.int64)
    lo = _lo(c, W, P, split)
    # exact integer restatement of the ranges
    if split == 0:
        ref = c * W // P
    else:
        h, j = P // 2, c // 2
        a, b = j * W // h, (j + 1) * W // h
        ref = np.where(c % 2 == 0, a, a + (b - a) * split // 256)
    np.testing.assert_array_equal(lo, ref)
    assert lo[0] == 0 and lo[-1] == W and (np.diff(lo) >= 0).all()
    # owner(p) is the chunk holding window p: every window of a small map, a sample of a large one
    p = np.arange(W, dtype=np.int64) if W <= 1 << 16 else np.unique(np.concatenate([
        np.random.default_rng(2).integers(0, W, 1 << 16), lo[1:-1] - 1, lo[1:-1], [0, W - 1]]))
    p = p[(p >= 0) & (p < W)]
    own = _owner(p, W, P, split)
    assert ((own >= 0) & (own < P)).all()
    assert (lo[own] <= p).all() and (p < lo[own + 1]).all()
