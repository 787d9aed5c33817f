"""Accuracy of the register backward's recovered positions (CPU emulation).

The register backward (nstepsolver 50, no adaptive substeps) keeps only the
cells of phase 1 and recovers each earlier position from the next through the
cell's inverse one-step map.  A recovered position's rounding is carried one
step back multiplied by M_c, so the kernels recover positions only for rows
whose bound (max_c ||M_c||_2)^50 is at most 16 and replay the others from
checkpoints.  These tests emulate the recovery on the oracle's replayed
trajectories (`helpers.recover_error`) and pin the error it admits on each
side of that bound."""
import numpy as np
import pytest

from oracle import oracle as orc

from helpers import cpab_for, recover_error, recover_growth, seeded_theta, uniform_points

# The library's bound on (max_c ||M_c||_2)^T for recovering positions.
RECOVER_GROWTH = 16.0


def _case(tess, scale, seed, n_theta=6, nP=1500):
    T = cpab_for(tess)
    p = T.params
    nd = len(tess)
    theta = seeded_theta(T, n_theta, scale, seed)
    As = orc.affine(theta, p.basis).reshape(n_theta, p.nC, nd, nd + 1)
    pts = uniform_points(nd, nP, seed + 1)
    return recover_growth(As), recover_error(pts, As, p.nc)


@pytest.mark.parametrize("tess,scales", [([10, 10], (0.5, 1.0, 1.5)), ([20, 20], (0.5, 1.0)),
                                         ([6], (1.0, 2.0, 3.0)), ([3, 3, 3], (1.0, 2.0, 3.0))])
def test_recovered_positions_within_bound(tess, scales):
    # Sampled over many rows (1D/2D/3D, growth 1 .. 16): the largest error is
    # ~4e-6 below growth 2 (theta ~ N(0, 0.5^2), the benchmark scale), ~7e-6
    # below 8 and 1.1e-5 .. 1.5e-5 between 8 and 16.
    rows = []
    for k, scale in enumerate(scales):
        g, e = _case(tess, scale, 300 + 10 * k)
        rows += list(zip(g, e))
    rows = np.array(rows)
    inside = rows[rows[:, 0] <= RECOVER_GROWTH]
    assert len(inside) >= 6, rows
    assert inside[:, 1].max() <= 2e-5, inside
    assert rows[rows[:, 0] <= 2.5, 1].max(initial=0.0) <= 6e-6, rows
    assert rows[rows[:, 0] <= 8.0, 1].max(initial=0.0) <= 1e-5, rows


def test_recovery_error_grows_beyond_bound():
    # Stronger fields (growth 1e2 .. 1e3) amplify the rounding by far more:
    # the reason such rows replay from checkpoints instead.
    g, e = _case([20, 20], 3.0, 400)
    assert (g > 50.0).all(), g
    assert e.max() >= 2.5e-5, (g, e)
