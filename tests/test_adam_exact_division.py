"""The Adam kernel divides by a per-tensor constant (b1t, b2t), by a block's
absmax and by 127 through a double-precision product with the divisor's
double reciprocal, rounded once to float.  That is the IEEE float quotient
bit for bit: an exact quotient of two floats is never a float midpoint and
lies at least 2^-49 (relative) away from every midpoint, while
RN_d(x * RN_d(1/y)) is within 2^-52 of x/y, so rounding it to float lands on
RN_f(x/y) -- for quotients in the normal float range.  A subnormal quotient
has fewer bits and can be a float midpoint, where the product may round the
other way: the kernel sends those to a float division (m / b1t) or uses the
quotient only where it rounds to code 0 (x / absmax * 127).  These tests
check the claim (numpy's float32 division is IEEE), pin its boundary with a
subnormal counterexample, and plant a mistake in the claim's own terms (a
float reciprocal instead of a double one) to show that they can fail."""
import numpy as np


def _via_double(x, y):
    inv = 1.0 / y.astype(np.float64)
    return (x.astype(np.float64) * inv).astype(np.float32)


def _ieee(x, y):
    with np.errstate(all="ignore"):
        return (x / y).astype(np.float32)


def test_every_int8_code_over_127():
    # the dequantization c / 127 (optim.rs:98-100), c = (i8) byte: all 256 codes
    c = np.arange(-128, 128, dtype=np.float32)
    got = (c.astype(np.float64) * (1.0 / 127.0)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), _ieee(c, np.float32(127.0)).view(np.uint32))


def _random_floats(rng, n, lo_exp, hi_exp):
    mant = rng.integers(1 << 23, 1 << 24, n, dtype=np.int64).astype(np.float64)
    e = rng.integers(lo_exp, hi_exp, n)
    s = np.where(rng.integers(0, 2, n) == 1, -1.0, 1.0)
    return (s * np.ldexp(mant, e - 23)).astype(np.float32)


def test_random_quotients_match_ieee_division():
    rng = np.random.default_rng(0xD1F)
    total = 0
    for _ in range(8):
        n = 2_000_000
        # numerators across the Adam state's range, divisors in (0, 1] like
        # b1t / b2t and across a wide absmax range
        x = _random_floats(rng, n, -60, 20)
        for y in (np.abs(_random_floats(rng, n, -20, 1)), np.abs(_random_floats(rng, n, -60, 20))):
            y = np.where(y == 0, np.float32(1.0), y)
            want = _ieee(x, y)
            assert np.array_equal(_via_double(x, y).view(np.uint32), want.view(np.uint32))
            total += n
    assert total == 32_000_000


def test_near_midpoint_and_subnormal_quotients():
    # quotients that land next to float midpoints (x = y * (q + ulp/2) rounded)
    # and quotients in the subnormal range
    rng = np.random.default_rng(7)
    n = 1_000_000
    y = np.abs(_random_floats(rng, n, -8, 8)) + np.float32(1e-3)
    q = _random_floats(rng, n, -10, 10).astype(np.float64)
    half = np.ldexp(np.ones(n), np.frexp(q)[1] - 25)
    x = ((q + half) * y.astype(np.float64)).astype(np.float32)
    assert np.array_equal(_via_double(x, y).view(np.uint32), _ieee(x, y).view(np.uint32))
    xs = _random_floats(rng, n, -140, -120)
    ys = np.abs(_random_floats(rng, n, 0, 12)) + np.float32(1.0)
    assert np.array_equal(_via_double(xs, ys).view(np.uint32), _ieee(xs, ys).view(np.uint32))


def test_a_float_reciprocal_would_not_be_exact():
    # the same product with a float reciprocal differs from the division:
    # the tests above can see a wrong method
    rng = np.random.default_rng(11)
    x = _random_floats(rng, 100_000, -10, 10)
    y = np.abs(_random_floats(rng, 100_000, -10, 10))
    wrong = (x * (np.float32(1.0) / y)).astype(np.float32)
    assert not np.array_equal(wrong.view(np.uint32), _ieee(x, y).view(np.uint32))


def test_subnormal_quotient_can_be_a_midpoint():
    # 147 * 2^-149 / 98 = 1.5 * 2^-149, a midpoint: IEEE rounds to even (2),
    # the double product falls just below it (1).  The claim stops at the
    # normal range, and a subnormal quotient of m / b1t takes the kernel's
    # float division.
    x = np.array([147 * 2.0 ** -149], np.float32)
    y = np.array([98.0], np.float32)
    assert _ieee(x, y).view(np.uint32)[0] == 2
    assert _via_double(x, y).view(np.uint32)[0] == 1
    # and quantization: any subnormal quotient times 127 rounds to code 0
    q = np.float32(np.nextafter(np.float32(2.0 ** -126), np.float32(0)))
    assert abs(float(np.float32(q * np.float32(127.0)))) < 0.5
