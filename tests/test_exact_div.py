"""The kernels divide by the temperature as a multiply: d / t in float32 is
taken as (float)((double)d * (1.0 / (double)t)).  A quotient of two float32
values is never a midpoint between floats and lies at least about 2^-49
(relative) from every one, while the double product is within 2^-52 of it,
so both round to the same float.  Checked here against IEEE division (numpy
float32) on random bit patterns, subnormals, logit-gap / temperature ranges
and divisors near 1."""
import numpy as np


def _check(a, b):
    b = np.where(b == 0, np.float32(1), b).astype(np.float32)
    with np.errstate(all="ignore"):
        want = a / b
        got = (a.astype(np.float64) * (1.0 / b.astype(np.float64))).astype(np.float32)
    same = (want.view(np.uint32) == got.view(np.uint32)) | (np.isnan(want) & np.isnan(got))
    assert same.all(), (a[~same][:5], b[~same][:5])


def test_reciprocal_multiply_matches_division():
    rng = np.random.default_rng(11)
    n = 4_000_000
    bits = lambda: rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    _check(bits().view(np.float32), bits().view(np.float32))
    _check((bits() & np.uint32(0x80FFFFFF)).view(np.float32), (bits() & np.uint32(0x7FFFFFFF)).view(np.float32))
    gaps = -(rng.random(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    temps = ((1 + rng.random(n)) * 2.0 ** rng.integers(-17, 13, n)).astype(np.float32)
    _check(gaps, temps)
    near1 = (np.uint32(0x3F800000) - np.uint32(0x1000000) + (bits() % np.uint32(0x2000000))).view(np.float32)
    _check(bits().view(np.float32), near1)
    # special values: zeros, infinities, NaN, the smallest subnormal, the largest float
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4028235e38, 1e-5, 1.0], np.float32)
    A, Bv = np.meshgrid(sp, sp)
    _check(A.ravel(), Bv.ravel())
