"""CPU checks of the lookups' edge handling (cpab_device.hpp, cell_2d and cell_3d).

- The 2D edge test: the device decides "some coordinate outside
  (0, kClampHi]" from the bit patterns, (bits(x) - 1) as an unsigned integer
  >= bits(kClampHi).  Compared with the float compares it replaces,
  !(x > 0) | !(x <= kClampHi), over every pattern in the ranges where they
  could disagree (zeros, denormals, the clamp bound and 1, the top of the
  finite range, infinities and NaNs of both signs) and a random sample of the
  rest.
- The 2D edge path's form of the reference's out-of-domain rules (side rules
  as substituted local coordinates, the corner rule on lane masks), restated
  per lane, against the oracle's if-chain on the edge lattice, NaN / infinity
  combinations, points around the domain and points far outside it.
- The 3D corner prefilter: a positive corner overshoot only outside [+0, 1].
"""
import numpy as np
import pytest

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


# ---------------------------------------------------------------------------
# The 2D lookup's edge path (cpab_device.hpp, cell_2d): the inside rule on the
# clamped coordinates, with the side rules entered as substituted local
# coordinates (lx = -4 left, 4 right; ly = -2 bottom, 2 top) and lanes beyond
# a corner decided by the corner rule.  Restated per lane in numpy (a lane's
# bit of each mask), against the oracle's if-chain of the reference rules.
# ---------------------------------------------------------------------------

def _fma32(a, b, c):
    """float32 fma: the exact a*b + c (float64 holds these products exactly) rounded once."""
    return (np.float64(a) * np.float64(b) + np.float64(c)).astype(np.float32)


def _edge_rule_2d(px, py, nx, ny):
    fx, fy = np.float32(nx), np.float32(ny)

    def clamp(v):   # v_med3_f32(v, 0, K): NaN -> min3 -> 0
        return np.where(np.isnan(v), np.float32(0), np.minimum(np.maximum(v, np.float32(0)), K))

    with np.errstate(invalid="ignore"):
        xc, yc = clamp(px), clamp(py)
        sx, sy = np.floor(xc * fx), np.floor(yc * fy)
        lx, ly = _fma32(xc, fx, -sx), _fma32(yc, fy, -sy)
        square = (sy * fx + sx).astype(np.int64)
        xl, xh, yl, yh = px <= 0, px >= 1, py <= 0, py >= 1
        lxs = np.where(xl, np.float32(-4), np.where(xh, np.float32(4), lx)).astype(np.float32)
        lys = np.where(yl, np.float32(-2), np.where(yh, np.float32(2), ly)).astype(np.float32)
        m3 = lxs < lys
        m1 = (np.float32(1) - lxs) < lys
        corner = (xl | xh) & (yl | yh)
        pxfx, pyfy = px * fx, py * fy
        xhi = _fma32(px, fx, np.full_like(px, -fx))
        yhi = _fma32(py, fy, np.full_like(py, -fy))
        lhs = np.where(yl, np.where(xl, pxfx, -xhi), yhi)
        rhs = np.where(yl, pyfy, np.where(xl, -pxfx, xhi))
        y_wins = (lhs > rhs) & corner
    m3 = (m3 & ~y_wins) | (y_wins & yh)
    m1 = (m1 & ~y_wins) | (y_wins & yh)
    return (4 * square + 2 * m3 + (m3 ^ m1)).astype(np.int32)


@pytest.mark.parametrize("tess", [[20, 20], [30, 30], [3, 5], [16, 16], [1, 1], [1000, 7]])
def test_edge_rule_matches_reference_rules(tess):
    from oracle import oracle as orc
    from helpers import edge_lattice
    rng = np.random.default_rng(3)
    special = np.array([np.nan, -np.nan, np.inf, -np.inf], np.float32)
    lat = edge_lattice(tess, 31)
    sp = np.stack(np.meshgrid(np.concatenate([special, lat[0, :40]]),
                              np.concatenate([special, lat[1, :40]]), indexing="ij")).reshape(2, -1)
    wide = (rng.random((2, 200000)) * 1.6 - 0.3).astype(np.float32)
    far = (rng.standard_normal((2, 100000)) * 1e3).astype(np.float32)
    for pts in (lat, sp.astype(np.float32), wide, far):
        got = _edge_rule_2d(pts[0], pts[1], *tess)
        ref = orc.cells(2, pts, tess)
        bad = np.flatnonzero(got != ref)
        assert bad.size == 0, (pts[:, bad[:5]].T.tolist(), got[bad[:5]], ref[bad[:5]])


def test_corner_prefilter_3d():
    # cell_3d computes the corner rule's overshoots (|p - 1/2| - 1/2) * n only
    # when some lane has all three coordinates' bit patterns above 1.0's
    # (outside [+0, 1]): an overshoot is positive only there.
    # Patterns: +0 and the smallest values, [1/8, 2), the top of the range with
    # inf and NaN, -0 and negative denormals, (-2, -1/8], -inf and negative
    # NaNs, and a random sample of all patterns.
    spans = [(0, 1 << 24), (0x3e000000, 0x40000000), (0x7f000000, 0x80000000 + (1 << 24)),
             (0xbe000000, 0xc0000000), (0xff000000, 1 << 32)]
    rng = np.random.default_rng(5)
    sample = rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    chunks = [sample] + [np.arange(a, min(a + (1 << 24), hi), dtype=np.uint64).astype(np.uint32)
                         for lo, hi in spans for a in range(lo, hi, 1 << 24)]
    for u in chunks:
        x = u.view(np.float32)
        outside = u > np.uint32(0x3f800000)
        for n in (1, 10, 1000):
            with np.errstate(invalid="ignore", over="ignore"):
                pos = (np.abs(x - np.float32(0.5)) - np.float32(0.5)) * np.float32(n) > 0
            assert not np.any(pos & ~outside), n

