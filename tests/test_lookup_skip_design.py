"""Why the integrators run the full cell lookup at every step (CPU, oracle
trajectories).

A lane may skip a step's lookup when its point is provably still inside its
cell: the distance from its position at the last lookup to the cell's edges
exceeds the displacement accumulated since.  A wave of 64 lanes skips only when
every lane may, since a skipped lookup that any lane needs is executed by the
whole wave.  Along the C2 (random points), C3 (16 x 4 pixel walk tiles) and C5
(meshgrid rows) trajectories, even with every lane's bound refreshed whenever
its wave looks up, each lane needs a lookup at ~2 % of steps and whole waves
may skip at most ~30 % of them.  The skip test (accumulate the step length,
compare, ballot) costs ~4 VALU ops at every step, the 2D lookup ~15: at a 20-30 %
skip rate the saving (3-4.5 ops) does not pay for the test.  This test keeps
that premise checked; it measures nothing on the GPU.
"""
import numpy as np

import bench
from oracle import oracle as orc

from helpers import cpab_for, meshgrid


def _trajectories(tess, pts, theta, T=50):
    """Positions [T+1, 2, nP] (float64 from the oracle's fp32 cells and maps)."""
    p = cpab_for(tess).params
    As = orc.affine(theta[None], p.basis).reshape(1, p.nC, 2, 3)
    Tr = orc.expm(2, As, 1.0 / T)
    _, cells = orc.forward_trels(pts, Tr, As, p.nc, T, return_cells=True)
    cells = cells[0]
    M = Tr[0].astype(np.float64)
    P = np.empty((T + 1, 2, pts.shape[1]))
    P[0] = pts
    for t in range(T):
        c, x = cells[:, t], P[t]
        P[t + 1, 0] = M[c, 0, 0] * x[0] + M[c, 0, 1] * x[1] + M[c, 0, 2]
        P[t + 1, 1] = M[c, 1, 0] * x[0] + M[c, 1, 1] * x[1] + M[c, 1, 2]
    return P


def _edge_distance(x, y, n):
    """Distance to the nearest of the square's sides and diagonals (a lower
    bound on the distance to the edges of the point's triangle)."""
    xs, ys = x * n, y * n
    lx, ly = xs - np.floor(xs), ys - np.floor(ys)
    side = np.minimum(np.minimum(lx, 1 - lx), np.minimum(ly, 1 - ly)) / n
    diag = np.minimum(np.abs(lx - ly), np.abs(lx + ly - 1)) / np.sqrt(2) / n
    return np.minimum(side, diag)


def _skip_rates(P, n):
    """(fraction of wave-steps every lane may skip, per-lane lookup rate)."""
    T = P.shape[0] - 1
    W = P.shape[2] // 64
    X = P[:, 0, :W * 64].reshape(T + 1, W, 64)
    Y = P[:, 1, :W * 64].reshape(T + 1, W, 64)
    d = _edge_distance(X[0], Y[0], n)
    D = np.zeros_like(d)
    skips, lane_need = 0, 0.0
    for t in range(1, T):
        D = D + np.hypot(X[t] - X[t - 1], Y[t] - Y[t - 1])
        need = D >= d - 1e-6
        lane_need += need.mean()
        wave = need.any(axis=1)
        skips += int((~wave).sum())
        d = np.where(wave[:, None], _edge_distance(X[t], Y[t], n), d)
        D = np.where(wave[:, None], 0.0, D)
    return skips / (W * (T - 1)), lane_need / (T - 1)


def test_wave_level_lookup_skip_is_rare():
    rng = np.random.default_rng(0)
    rates = {}
    # C2: uniform random points, [20, 20], theta scale 0.5
    T2 = cpab_for([20, 20])
    pts = rng.random((2, 64 * 120)).astype(np.float32)
    rates["c2"] = _skip_rates(_trajectories([20, 20], pts, bench._theta(T2, 1, 0.5, 11)[0]), 20)
    # C5 stage: rows of the 512 x 512 meshgrid (64 lanes along x), [16, 16], scale 0.3
    T5 = cpab_for([16, 16])
    th5 = (np.random.default_rng(51).standard_normal(T5.params.d) * 0.3).astype(np.float32)
    g = meshgrid([512, 512])
    rows = rng.choice(512, 12, replace=False)
    sel = np.concatenate([np.arange(r * 512, (r + 1) * 512) for r in rows])
    rates["c5"] = _skip_rates(_trajectories([16, 16], g[:, sel].astype(np.float32), th5), 16)
    # C3: 16 x 4 walk tiles of the 512 x 512 image, [30, 30], scale 0.5
    T3 = cpab_for([30, 30])
    pts3 = []
    for a in rng.choice(np.arange(0, 512, 4), 12):
        for b in rng.choice(np.arange(0, 512, 16), 12):
            for k in range(4):
                for l in range(16):
                    pts3.append(((a + k) / 511.0, (b + l) / 511.0))
    pts3 = np.array(pts3, np.float32).T.copy()
    rates["c3"] = _skip_rates(_trajectories([30, 30], pts3, bench._theta(T3, 1, 0.5, 33)[0]), 30)
    for name, (wave_skip, lane_need) in rates.items():
        assert lane_need < 0.05, (name, lane_need)
        assert wave_skip < 0.4, (name, wave_skip)
