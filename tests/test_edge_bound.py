"""CPU checks of the 2D domain-edge bound (fg-cpab_amd/csrc/cpab_device.hpp,
edge_bound_cell_2d and edge_delta_2d; restated in tests/edge_bound.py).

The backward's replay skips the lookup's per-step domain-edge test for a wave
whose lanes all start at distance >= delta_T from every edge of the domain,
on the claim that such trajectories stay in (0, 1 - 2^-23]^2 for all T
computed explicit-midpoint steps.  These tests check that claim against the
oracle's fp32 replay trajectories (the positions every step looks up), for
points placed at and just beyond delta_T from each edge and corner, at the
benchmark's field strength and at much stronger ones, with zero-boundary and
general bases.
They also check that the bound is not vacuous at the benchmark's strength
(most waves of a random point set qualify), that unusable maps give no bound,
and the closed form against the step-by-step recursion it stands for."""
import numpy as np
import pytest

from cpab import Cpab
from oracle import oracle as orc
import edge_bound as eb
from helpers import cpab_for, seeded_theta, uniform_points

K = np.float32(1.0 - 1e-7)


def _inside(path):
    """[..., 2, nP] positions -> [..., nP] inside (0, kClampHi]^2."""
    with np.errstate(invalid="ignore"):
        return ((path > 0) & (path <= K)).all(axis=-2)


def _probe_points(delta, rng, n_rand=4000):
    """Random points, and points at 1x, 1.01x, 2x and 10x delta from each edge and corner."""
    pts = [rng.random((2, n_rand)).astype(np.float32)]
    for f in (1.0, 1.01, 2.0, 10.0):
        d = np.float32(min(delta * f, 0.25))
        u = rng.random(256).astype(np.float32)
        for fixed_axis, val in ((0, d), (0, np.float32(1) - d), (1, d), (1, np.float32(1) - d)):
            q = np.empty((2, 256), np.float32)
            q[fixed_axis] = val
            q[1 - fixed_axis] = u
            pts.append(q)
        for cx in (d, np.float32(1) - d):
            for cy in (d, np.float32(1) - d):
                pts.append(np.array([[cx] * 4, [cy] * 4], np.float32))
    return np.concatenate(pts, axis=1)


def _check_rows(T_cpab, theta, nstep, rng):
    p = T_cpab.params
    nx, ny = p.nc
    As = orc.affine(theta, p.basis).reshape(theta.shape[0], -1, 2, 3).astype(np.float32)
    deltas = []
    for b in range(theta.shape[0]):
        delta = eb.midpoint_delta(As[b], nstep, nx, ny)
        deltas.append(delta)
        if not np.isfinite(delta):
            continue
        pts = _probe_points(float(delta), rng)
        safe = eb.safe_start(pts, delta)
        assert safe.sum() > 0
        _, path = orc.forward_midpoint(pts, As[b:b + 1], [nx, ny], nstep, return_path=True)
        ok = _inside(path[0]).all(axis=0)         # every looked-up position inside
        bad = np.flatnonzero(safe & ~ok)
        assert bad.size == 0, (b, float(delta), pts[:, bad[:4]].T.tolist())
    return np.array(deltas)


@pytest.mark.parametrize("tess,scale", [([20, 20], 0.5), ([6, 5], 0.5), ([6, 5], 2.0),
                                        ([6, 5], 5.0), ([3, 4], 10.0), ([16, 16], 1.5)])
def test_bound_holds_on_oracle_trajectories(tess, scale):
    T = cpab_for(tess)
    rng = np.random.default_rng(7 + int(scale * 10))
    theta = seeded_theta(T, 4, scale, 500 + len(tess) * 10 + int(scale * 10))
    deltas = _check_rows(T, theta, 50, rng)
    if scale <= 0.5:
        # at the benchmark's strength every row has a bound, and a small one
        assert np.isfinite(deltas).all() and deltas.max() < 1e-3, deltas


def test_bound_holds_with_other_step_counts():
    T = cpab_for([5, 4])
    rng = np.random.default_rng(11)
    for nstep in (10, 37, 100):
        _check_rows(T, seeded_theta(T, 3, 1.0, 600 + nstep), nstep, rng)


@pytest.mark.parametrize("scale", [0.3, 1.0, 5.0])
def test_bound_holds_for_general_bases(scale):
    # Without zero boundary the fields carry points across the domain's edges:
    # the bound, where it exists, only admits points far enough inside.
    T = Cpab([4, 4], zero_boundary=False)
    rng = np.random.default_rng(13)
    deltas = _check_rows(T, seeded_theta(T, 4, scale, 700 + int(scale * 10)), 50, rng)
    assert (deltas > 1e-3).all(), deltas


def test_most_random_waves_qualify_at_benchmark_strength():
    # C2's shape: 64 uniform points per wave, theta ~ N(0, 0.5^2): nearly every
    # wave starts beyond delta_T of every edge and may skip the edge test.
    T = cpab_for([20, 20])
    theta = seeded_theta(T, 2, 0.5, 22)
    As = orc.affine(theta, T.params.basis).reshape(2, -1, 2, 3).astype(np.float32)
    pts = uniform_points(2, 64 * 4000, 21)
    for b in range(2):
        delta = eb.midpoint_delta(As[b], 50, 20, 20)
        waves = eb.safe_start(pts, delta).reshape(-1, 64).all(axis=1)
        assert waves.mean() > 0.9, (float(delta), waves.mean())


def _fields(A_row):
    return np.tile(np.array(A_row, np.float32), (16, 1))


def test_unusable_maps_give_no_bound():
    zero = [0, 0, 0, 0, 0, 0]
    assert np.isfinite(eb.midpoint_delta(_fields(zero), 50, 2, 2))
    for bad in (np.inf, np.nan):
        f = _fields(zero)
        f[0, 1] = bad
        assert not np.isfinite(eb.midpoint_delta(f, 50, 2, 2))
    # a field that pushes points out of the domain: no alpha > 0
    assert not np.isfinite(eb.midpoint_delta(_fields([0, 0, -40, 0, 0, 0]), 50, 2, 2))


def test_zero_field_gives_the_margins():
    # The zero field leaves every point where it is: delta is the edge
    # threshold 2^-23 plus T - 1 steps of the margins, the cell-assignment
    # margin 2 * 2^-20 (beta's slope + 1 at alpha = 1) and the rounding bound.
    h = np.float32(1.0) / np.float32(50)
    per_step = 2 * eb.ETA + eb.midpoint_step_err(np.zeros(6, np.float32), float(h), float(h / 2))
    d = float(eb.midpoint_delta(_fields([0, 0, 0, 0, 0, 0]), 50, 2, 2))
    assert 2.0 ** -23 + 49 * per_step <= d < (2.0 ** -23 + 49 * per_step) * 1.001, d


def test_closed_form_covers_the_recursion():
    # delta_T = (thr + (T-1) b) / m^(T-1) is at least the step-by-step
    # threshold max(thr, (delta + b) / alpha) the argument needs.
    for al in (0.5, 0.9, 0.99, 1.0, 1.2):
        for b in (0.0, 1e-9, 1e-6):
            for T in (1, 2, 10, 50, 100):
                thr, dl = 2.0 ** -23, 2.0 ** -23
                for _ in range(1, T):
                    dl = max(thr, (dl + b) / al)
                closed = (thr + (T - 1) * b) * eb.pow_int(1.0 / min(al, 1.0), T - 1)
                assert closed >= dl * (1 - 1e-12), (al, b, T, closed, dl)
