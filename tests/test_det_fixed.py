"""The deterministic backward's float -> 64-bit fixed-point conversion
(det_fixed in fg-cpab_amd/csrc/cpab_device.hpp), restated op by op in numpy
float32 and checked against the exact integer rint(v * 2^s) computed with
Python integers, over magnitudes up to the 2^62 the scale allows, both signs,
ties and values that round to zero."""
import numpy as np

F = np.float32


def det_fixed(v, s):
    x = np.rint(np.ldexp(F(v), s).astype(F))           # v * 2^s exact; rintf (ties to even)
    a = np.abs(x)
    hi = np.floor(a * F(2.0 ** -32))
    lo = F(np.float64(-hi) * 2.0 ** 32 + np.float64(a))  # fmaf: exact, then one rounding
    u = (int(hi) << 32) | int(lo)
    assert int(lo) == lo and 0 <= int(lo) < 2 ** 32 and int(hi) == hi
    return -u if x < 0 else u


def exact(v, s):
    from fractions import Fraction
    q = Fraction(float(v)) * (Fraction(2) ** s)
    f = q.numerator // q.denominator
    r = q - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        f += 1
    return f


def test_det_fixed_matches_exact_rounding():
    rng = np.random.default_rng(7)
    cases = [(F(0.5), 0), (F(1.5), 0), (F(2.5), 0), (F(-0.5), 0), (F(-1.5), 0), (F(-2.5), 0),
             (F(1.0), 61), (F(-1.0), 61), (F(-1e-30), 4), (F(3.0), -2), (F(-3.0), -2)]
    for _ in range(4000):
        e = int(rng.integers(-40, 40))
        v = F(rng.standard_normal() * 2.0 ** e)
        # the scale keeps |v| 2^s below 2^62 for the row's largest value
        _, ve = np.frexp(np.abs(v) if v != 0 else F(1.0))
        s = int(rng.integers(-10, 62 - int(ve) + 1))
        cases.append((v, s))
    for v, s in cases:
        assert det_fixed(v, s) == exact(v, s), (v, s)


def test_det_fixed_large_and_negative_split():
    # magnitudes at or above 2^32 split into a high word and a low word that is a
    # multiple of the value's ulp; negative values negate the 64-bit magnitude
    for v in (F(2.0 ** 40 + 2.0 ** 20), F(-(2.0 ** 40 + 2.0 ** 20)), F(2.0 ** 61 * 1.75),
              F(-(2.0 ** 61 * 1.75)), F(2.0 ** 32), F(-(2.0 ** 32)), F(4294967040.0)):
        assert det_fixed(v, 0) == int(v)
