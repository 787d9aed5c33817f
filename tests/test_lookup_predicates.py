"""CPU check of the 2D lookup's edge test (cpab_device.hpp, cell_2d).

The device decides "some coordinate outside (0, kClampHi]" from the bit
patterns: (bits(x) - 1) as an unsigned integer >= bits(kClampHi).  This test
compares that predicate with the float compares it replaces,
!(x > 0) | !(x <= kClampHi), over every pattern in the ranges where they could
disagree (zeros, denormals, the clamp bound and 1, the top of the finite range,
infinities and NaNs of both signs) and a random sample of the rest.
"""
import numpy as np

K = np.float32(1.0 - 1e-7)   # kClampHi: rounds to 1 - 2^-23


def _check(u):
    u = np.asarray(u, dtype=np.uint32)
    x = u.view(np.float32)
    with np.errstate(invalid="ignore"):
        ref = ~(x > 0) | ~(x <= K)
    dev = (u - np.uint32(1)) >= K.view(np.uint32)
    bad = np.flatnonzero(ref != dev)
    assert bad.size == 0, [hex(int(v)) for v in u[bad[:8]]]


def test_clamp_bound_value():
    assert K.view(np.uint32) == np.float32(1.0).view(np.uint32) - 2


def test_edge_predicate_matches_float_compares():
    kb = int(K.view(np.uint32))
    spans = [(0, 1 << 24),                                     # +0, denormals, small normals
             (kb - (1 << 20), kb + (1 << 20)),                 # around the clamp bound and 1.0
             (0x7f000000, 0x80000000 + (1 << 24)),             # top of the range, inf, NaN, -0, -denormals
             (0xbf000000, 0xbf800000 + (1 << 20)),             # around -1
             (0xff000000, 1 << 32)]                            # -inf and negative NaNs
    for lo, hi in spans:
        for a in range(lo, hi, 1 << 24):
            _check(np.arange(a, min(a + (1 << 24), hi), dtype=np.uint64))
    rng = np.random.default_rng(7)
    _check(rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64))
