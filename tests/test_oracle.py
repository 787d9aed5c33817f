"""Pins the CPU oracle (oracle/) against what the mathematics fixes, so that a
plausible slip in the restatement (a dropped term, a sign, a transposed index)
fails here.  The reference ships no tests or golden vectors for this path, so
the anchors are: scipy's expm, the exact flow of a cell-independent field,
the analytic 1D ODE solution, barycentric containment of the looked-up cell,
finite differences of the float64 midpoint scheme for the adjoint, the theta=0
closed form of the moments, dense B products, and textbook / torch bilinear
sampling.  CPU only."""
import numpy as np
import pytest
import scipy.linalg as sla
from scipy.integrate import solve_ivp

from oracle import oracle as orc

from helpers import cpab_for, meshgrid, scatter_magnitude, uniform_points


def _random_As(nC, nd, scale, seed, dtype=np.float32):
    return (np.random.default_rng(seed).standard_normal((1, nC, nd, nd + 1)) * scale).astype(dtype)


def _aug(A):
    nd = A.shape[0]
    M = np.zeros((nd + 1, nd + 1))
    M[:nd] = A
    return M


@pytest.mark.parametrize("nd", [1, 2, 3])
@pytest.mark.parametrize("scale,dT,tol", [(1.0, 0.02, 2e-6), (3.0, 0.5, 5e-4), (30.0, 0.5, 2e-3)])
def test_expm_matches_scipy(nd, scale, dT, tol):
    # The larger norms take the scaling-and-squaring branch; each squaring
    # doubles the fp32 rounding error of the Pade approximant, hence the tolerances.
    A = (np.random.default_rng(nd).standard_normal((200, nd, nd + 1)) * scale).astype(np.float32)
    got = orc.expm(nd, A, dT)
    for i in range(200):
        ref = sla.expm(_aug(A[i].astype(np.float64)) * np.float32(dT))[:nd]
        np.testing.assert_allclose(got[i], ref, rtol=tol, atol=tol * np.abs(ref).max())


def test_expm_zero_is_identity():
    for nd in (1, 2, 3):
        out = orc.expm(nd, np.zeros((5, nd, nd + 1), np.float32), 0.02)
        ref = np.broadcast_to(np.eye(nd + 1)[:nd], out.shape)
        np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("nd,nc", [(2, [3, 4]), (3, [2, 3, 2])])
def test_trels_stepping_uniform_field_is_exact_flow(nd, nc):
    # The same A in every cell: T steps of expm(A/T) compose to expm(A), for
    # any cell sequence.  Pins apply() (row/column order) and the stepping.
    nC = 4 * nc[0] * nc[1] if nd == 2 else 5 * int(np.prod(nc))
    A = (np.random.default_rng(3).standard_normal((nd, nd + 1)) * 0.4).astype(np.float32)
    As = np.broadcast_to(A, (1, nC, nd, nd + 1)).copy()
    Tr = orc.expm(nd, As, 1.0 / 50)
    pts = uniform_points(nd, 500, 4)
    out = orc.forward_trels(pts, Tr, As, nc, 50)[0]
    ref = (sla.expm(_aug(A.astype(np.float64))) @ np.vstack([pts, np.ones(500)]))[:nd]
    np.testing.assert_allclose(out, ref, atol=2e-5)


def test_midpoint_uniform_field_second_order():
    # Explicit midpoint with uniform A: per step p <- (I + hA + h^2 A^2/2)p (+ b terms);
    # matches expm(A) up to O(h^2) and exactly its own truncated series.
    A = np.array([[0.3, -0.2, 0.05], [0.1, 0.25, -0.02]])
    As = np.broadcast_to(A, (1, 4 * 6, 2, 3)).copy()
    pts = uniform_points(2, 300, 5).astype(np.float64)
    out = orc.forward_midpoint(pts, As, [2, 3], 50, dtype=np.float64)[0]
    h = 1 / 50
    M = _aug(A)
    step = np.eye(3) + h * M + (h * h / 2) * M @ M
    ref = (np.linalg.matrix_power(step, 50) @ np.vstack([pts, np.ones(300)]))[:2]
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-13)


def test_1d_closed_form_matches_ode():
    T = cpab_for([7])
    As = _random_As(7, 1, 1.5, 9, np.float64)
    As = (np.asarray(T.params.basis @ (np.random.default_rng(2).standard_normal(T.params.d) * 1.5))
          .reshape(1, 7, 1, 2))
    pts = np.linspace(0.0, 1.0, 41)[None]
    got = orc.forward_closed_1d(pts.astype(np.float32), As.astype(np.float32), [7])[0, 0]
    A = As.astype(np.float32).astype(np.float64)[0, :, 0]

    def v(_, x):
        c = min(max(int(np.floor(min(max(x[0], 0.0), 1 - 1e-7) * 7)), 0), 6)
        return [A[c, 0] * x[0] + A[c, 1]]

    for i, x0 in enumerate(pts[0]):
        sol = solve_ivp(v, (0, 1), [x0], rtol=1e-11, atol=1e-12, max_step=0.01)
        assert abs(got[i] - sol.y[0, -1]) < 5e-6, (x0, got[i], sol.y[0, -1])


def test_1d_closed_form_is_monotone():
    T = cpab_for([50])
    th = np.random.default_rng(11).standard_normal((4, T.params.d)) * 0.5
    As = orc.affine(th.astype(np.float32), T.params.basis).reshape(4, 50, 1, 2)
    pts = np.linspace(0, 1, 5000, dtype=np.float32)[None]
    out = orc.forward_closed_1d(pts, As, [50])[:, 0]
    assert (np.diff(out, axis=1) >= 0).all()
    np.testing.assert_array_equal(out[:, 0], 0.0)
    np.testing.assert_array_equal(out[:, -1], 1.0)


def _barycentric_ok(verts, p, tol=1e-5):
    # verts rows are homogeneous vertices [x.., 1]; solve V^T w = [p; 1]
    w = np.linalg.solve(verts.T, np.append(p, 1.0))
    return (w >= -tol).all()


@pytest.mark.parametrize("tess", [[5, 4], [3, 3, 4], [2, 2, 2]])
def test_lookup_cell_contains_point(tess):
    T = cpab_for(tess)
    nd = len(tess)
    pts = uniform_points(nd, 4000, 17)
    cells = orc.cells(nd, pts, tess)
    V = T.tesselation.verts
    for i in range(pts.shape[1]):
        assert _barycentric_ok(V[cells[i]], pts[:, i].astype(np.float64)), (pts[:, i], cells[i])


@pytest.mark.parametrize("tess", [[4, 3], [3, 2, 2]])
def test_lookup_outside_uses_cell_of_boundary_projection(tess):
    # Outside the domain the cell must contain the point's projection onto the
    # domain boundary (up to ties along corner diagonals).
    T = cpab_for(tess)
    nd = len(tess)
    pts = (uniform_points(nd, 3000, 23) * 1.8 - 0.4).astype(np.float32)
    out = (pts < 0).any(0) | (pts > 1).any(0)
    cells = orc.cells(nd, pts, tess)
    V = T.tesselation.verts
    for i in np.flatnonzero(out):
        q = np.clip(pts[:, i].astype(np.float64), 0, 1)
        assert _barycentric_ok(V[cells[i]], q, tol=1e-5), (pts[:, i], cells[i])


@pytest.mark.parametrize("nd,tess,scale", [(1, [6], 1.0), (2, [3, 4], 1.0), (3, [2, 2, 3], 0.8)])
def test_adjoint_matches_finite_differences(nd, tess, scale):
    # d<g, phi_midpoint(p0; A)> / dA and / dp0 from the float64 backward versus
    # central differences of the float64 midpoint forward.
    T = cpab_for(tess)
    nC = T.params.nC
    rng = np.random.default_rng(40 + nd)
    As = (rng.standard_normal((2, nC, nd, nd + 1)) * scale)
    pts = 0.1 + 0.8 * rng.random((nd, 60))
    g = rng.standard_normal((2, nd, 60))
    mom, gp = orc.backward(pts, As, g, tess, 20, dtype=np.float64)
    dA = rng.standard_normal(As.shape)
    dp = rng.standard_normal(pts.shape)
    eps = 1e-6

    def L(A_, p_):
        return float((g * orc.forward_midpoint(p_, A_, tess, 20, dtype=np.float64)).sum())

    fd_A = (L(As + eps * dA, pts) - L(As - eps * dA, pts)) / (2 * eps)
    an_A = float((mom.reshape(As.shape) * dA).sum())
    assert abs(fd_A - an_A) <= 1e-6 * max(1.0, abs(an_A)), (fd_A, an_A)
    fd_p = (L(As, pts + eps * dp) - L(As, pts - eps * dp)) / (2 * eps)
    an_p = float((gp * dp[None]).sum())
    assert abs(fd_p - an_p) <= 1e-6 * max(1.0, abs(an_p)), (fd_p, an_p)


# ---- adaptive substeps (Heun correction on a cell crossing) -----------------
# cpab_ops_2d.cu:202-219 (Trels forward) and :294-332 (midpoint replay of the
# backward), cpab_ops_1d.cu:229-261, cpab_ops_3d.cu:209-225: a step whose
# endpoint q lies in another cell ce is replaced by p + (h/2) (A_c [p;1] +
# A_ce [q;1]).  Pinned below by an independent float64 evaluation of one step
# (T = 1, so h = 1) with a different field in every cell, by the identity of
# adaptive and plain stepping on trajectories that never cross, and by the
# order of the corrected step for a cell-independent field.

def _step_cases(nd):
    tess = {1: [6], 2: [4, 3], 3: [2, 3, 2]}[nd]
    nC = {1: 6, 2: 48, 3: 60}[nd]
    rng = np.random.default_rng(120 + nd)
    As = rng.standard_normal((1, nC, nd, nd + 1)) * {1: 0.25, 2: 0.25, 3: 0.06}[nd]
    pts = 0.05 + 0.9 * rng.random((nd, 400))
    return tess, As, pts


def _vel(A, p):
    """A [nP, nd, nd+1] applied to p [nd, nP]: velocity [nd, nP] (float64)."""
    return np.einsum("nij,jn->in", A[:, :, :-1], p) + A[:, :, -1].T


@pytest.mark.parametrize("nd", [1, 2, 3])
def test_adaptive_replay_step_closed_form(nd):
    tess, As, pts = _step_cases(nd)
    out = orc.forward_midpoint(pts, As, tess, 1, adaptive=True, dtype=np.float64)[0]
    c = orc.cells(nd, pts, tess)
    A0 = As[0, c]
    q = pts + _vel(A0, pts + 0.5 * _vel(A0, pts))   # explicit midpoint, h = 1
    ce = orc.cells(nd, q, tess)
    cross = ce != c
    heun = pts + 0.5 * (_vel(A0, pts) + _vel(As[0, ce], q))
    ref = np.where(cross[None], heun, q)
    assert 20 < cross.sum() < 380, cross.sum()   # both branches exercised
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-14)
    plain = orc.forward_midpoint(pts, As, tess, 1, adaptive=False, dtype=np.float64)[0]
    np.testing.assert_allclose(plain, q, rtol=0, atol=1e-14)
    assert np.abs(out - plain)[:, cross].max() > 1e-6   # the correction changes crossing steps


@pytest.mark.parametrize("nd", [2, 3])
def test_adaptive_trels_step_closed_form(nd):
    tess, As, pts = _step_cases(nd)
    Tr = np.stack([sla.expm(_aug(A))[:nd] for A in As[0]])[None]   # h = 1
    out = orc.forward_trels(pts, Tr, As, tess, 1, adaptive=True, dtype=np.float64)[0]
    c = orc.cells(nd, pts, tess)
    s = _vel(Tr[0, c], pts)   # the one-step map applied like a velocity: Tr [p; 1]
    ce = orc.cells(nd, s, tess)
    cross = ce != c
    heun = pts + 0.5 * (_vel(As[0, c], pts) + _vel(As[0, ce], s))
    ref = np.where(cross[None], heun, s)
    assert 20 < cross.sum() < 380, cross.sum()
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-13)


@pytest.mark.parametrize("nd,tess", [(1, [50]), (2, [20, 20]), (3, [4, 4, 4])])
def test_adaptive_identical_without_crossings(nd, tess):
    # Trajectories that never change cell take no correction: forward, replay
    # and backward (moments and point adjoints) are bit-identical with and
    # without adaptive substeps.  The backward's reverse sweep differentiates
    # the plain midpoint step in each visited cell either way, so with T = 1
    # (one step, at the start point) the two backwards agree even on crossings.
    T = cpab_for(tess)
    p = T.params
    th = (np.random.default_rng(130 + nd).standard_normal((2, p.d)) * 0.5).astype(np.float32)
    As = orc.affine(th, p.basis).reshape(2, p.nC, nd, nd + 1)
    pts = uniform_points(nd, 4000, 131)
    end, cl = orc.forward_midpoint(pts, As, tess, 50, return_cells=True)
    # no cell change under either theta, the last step's endpoint included
    still = ((cl == cl[:, :, :1]).all(axis=2) &
             (np.stack([orc.cells(nd, e, tess) for e in end]) == cl[:, :, 0])).all(axis=0)
    assert 100 < still.sum() < 4000
    q = np.ascontiguousarray(pts[:, still])
    g = np.random.default_rng(132).standard_normal((2, nd, q.shape[1])).astype(np.float32)
    np.testing.assert_array_equal(orc.forward_midpoint(q, As, tess, 50, adaptive=True),
                                  orc.forward_midpoint(q, As, tess, 50))
    m1, l1 = orc.backward(q, As, g, tess, 50, adaptive=True)
    m0, l0 = orc.backward(q, As, g, tess, 50)
    np.testing.assert_array_equal(m1, m0)
    np.testing.assert_array_equal(l1, l0)
    if nd > 1:
        Tr = orc.expm(nd, As, 1.0 / 50)
        end, ct = orc.forward_trels(pts, Tr, As, tess, 50, return_cells=True)
        keep = ((ct == ct[:, :, :1]).all(axis=2) &
                (np.stack([orc.cells(nd, e, tess) for e in end]) == ct[:, :, 0])).all(axis=0)
        fixed = np.ascontiguousarray(pts[:, keep])
        np.testing.assert_array_equal(orc.forward_trels(fixed, Tr, As, tess, 50, adaptive=True),
                                      orc.forward_trels(fixed, Tr, As, tess, 50))
    g_all = np.random.default_rng(133).standard_normal((2, nd, pts.shape[1])).astype(np.float32)
    m1, l1 = orc.backward(pts, As, g_all, tess, 1, adaptive=True)
    m0, l0 = orc.backward(pts, As, g_all, tess, 1)
    np.testing.assert_array_equal(m1, m0)
    np.testing.assert_array_equal(l1, l0)


def test_adaptive_uniform_field_order():
    # One field in every cell: a corrected step is trapezoidal with the exact
    # (Trels) or midpoint endpoint.  For linear fields that is
    #   Trels:    I + hM + h^2M^2/2 + h^3M^3/4 + ...   (exact flow: h^3 M^3 / 6)
    #   midpoint: I + hM + h^2M^2/2 + h^3M^3/4          (midpoint: no h^3 term)
    # so with k corrected steps the endpoint moves from the plain one by about
    # k h^3 ||M^3 p|| / 12 (Trels) or / 4 (midpoint), and never more.
    nd, tess, T = 2, [6, 6], 20
    A = np.array([[0.9, -1.3, 0.2], [1.1, 0.4, -0.3]])
    As = np.broadcast_to(A, (1, 4 * 36, 2, 3)).copy()
    pts = 0.2 + 0.6 * uniform_points(2, 500, 134).astype(np.float64)
    h = 1.0 / T
    M = _aug(A)
    ph = np.vstack([pts, np.ones(500)])
    bound = (h ** 3) * np.linalg.norm(np.linalg.matrix_power(M, 3), 2) * np.linalg.norm(ph, axis=0)
    Tr = np.broadcast_to(sla.expm(h * M)[:2], As.shape).copy()
    out_t, ct = orc.forward_trels(pts, Tr, As, tess, T, adaptive=True, return_cells=True,
                                  dtype=np.float64)
    plain_t = orc.forward_trels(pts, Tr, As, tess, T, dtype=np.float64)
    k = (np.diff(ct[0], axis=1) != 0).sum(axis=1) + 1   # steps that may have been corrected
    growth = np.exp(np.linalg.norm(M, 2))
    d = np.linalg.norm(out_t[0] - plain_t[0], axis=0)
    assert (d <= growth * k * bound / 12 * 1.01 + 1e-13).all()
    assert d.max() > 0
    out_m = orc.forward_midpoint(pts, As, tess, T, adaptive=True, dtype=np.float64)
    plain_m = orc.forward_midpoint(pts, As, tess, T, dtype=np.float64)
    d = np.linalg.norm(out_m[0] - plain_m[0], axis=0)
    assert (d <= growth * k * bound / 4 * 1.01 + 1e-13).all()
    assert d.max() > 0


def test_moments_closed_form_at_zero_theta():
    # theta = 0: lambda stays g and p stays p0, so M_c = sum_{n in c} g_n [p_n; 1]^T
    # (T*h = 1) and grad_points = g.
    tess = [5, 4]
    nC = 80
    pts = uniform_points(2, 3000, 50)
    g = np.random.default_rng(51).standard_normal((2, 2, 3000)).astype(np.float32)
    mom, gp = orc.backward(pts, np.zeros((2, nC, 2, 3), np.float32), g, tess, 50)
    np.testing.assert_array_equal(gp, g)
    cells = orc.cells(2, pts, tess)
    ph = np.vstack([pts, np.ones(3000)]).astype(np.float64)
    ref = np.zeros((2, nC, 2, 3))
    for b in range(2):
        for n in range(3000):
            ref[b, cells[n]] += np.outer(g[b, :, n], ph[:, n])
    np.testing.assert_allclose(mom.reshape(2, nC, 2, 3), ref, rtol=1e-5, atol=1e-5)


def test_backward_is_linear_in_grad_out():
    tess = [4, 4]
    As = _random_As(64, 2, 0.7, 60, np.float64).repeat(2, 0)
    pts = uniform_points(2, 500, 61).astype(np.float64)
    rng = np.random.default_rng(62)
    g1, g2 = rng.standard_normal((2, 2, 2, 500))
    m1, p1 = orc.backward(pts, As, g1, tess, 50, dtype=np.float64)
    m2, p2 = orc.backward(pts, As, g2, tess, 50, dtype=np.float64)
    m3, p3 = orc.backward(pts, As, 2 * g1 - 3 * g2, tess, 50, dtype=np.float64)
    np.testing.assert_allclose(m3, 2 * m1 - 3 * m2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(p3, 2 * p1 - 3 * p2, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("tess", [[50], [20, 20], [3, 3, 3]])
def test_affine_and_project_match_dense(tess):
    T = cpab_for(tess)
    B = T.params.basis.toarray()
    rng = np.random.default_rng(70)
    th = rng.standard_normal((3, B.shape[1])).astype(np.float32)
    np.testing.assert_allclose(orc.affine(th, T.params.basis), th.astype(np.float64) @ B.T,
                               rtol=1e-5, atol=1e-6)
    M = rng.standard_normal((3, B.shape[0])).astype(np.float32)
    np.testing.assert_allclose(orc.project(M, T.params.basis), M.astype(np.float64) @ B,
                               rtol=1e-5, atol=1e-5)
    # float64 twin is exact up to summation order
    np.testing.assert_allclose(orc.project(M.astype(np.float64), T.params.basis, dtype=np.float64),
                               M.astype(np.float64) @ B, rtol=1e-12, atol=1e-12)


def test_cycle_consistency():
    # T(T(x; theta); -theta) ~ x (rectangular_grid_diffeomorphism_2d.py:104-107)
    T = cpab_for([20, 20])
    th = (np.random.default_rng(80).standard_normal((2, T.params.d)) * 0.5).astype(np.float32)
    pts = uniform_points(2, 4000, 81)

    def fwd(p, t):
        As = orc.affine(t, T.params.basis).reshape(2, -1, 2, 3)
        return orc.forward_trels(p, orc.expm(2, As, 1 / 50), As, [20, 20], 50)

    back = fwd(fwd(pts, th), -th)
    assert np.abs(back - pts[None]).mean() < 2e-5


def test_interp_matches_textbook_bilinear():
    rng = np.random.default_rng(90)
    data = rng.random((2, 3, 9, 7)).astype(np.float32)
    grid = (rng.random((2, 2, 5 * 6)) * 1.4 - 0.2).astype(np.float32)
    out = orc.interp_forward(2, data, grid, (5, 6))
    for b in range(2):
        for p in range(30):
            i0, i1 = p % 5, p // 5
            x = np.clip(grid[b, 0, p] * 8, 0, 8)
            y = np.clip(grid[b, 1, p] * 6, 0, 6)
            x0, y0 = min(int(np.floor(x)), 7), min(int(np.floor(y)), 5)
            tx, ty = x - x0, y - y0
            v = ((1 - tx) * (1 - ty) * data[b, :, x0, y0] + tx * (1 - ty) * data[b, :, x0 + 1, y0]
                 + (1 - tx) * ty * data[b, :, x0, y0 + 1] + tx * ty * data[b, :, x0 + 1, y0 + 1])
            np.testing.assert_allclose(out[b, :, i0, i1], v, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("nd", [1, 2, 3])
def test_scatter_magnitude(nd):
    # The grad_data tolerance scale of the GPU tests.  Points inside [0, 1]
    # have weights in [0, 1], so it equals the float64 scatter of |gout|;
    # clamped points add cancelling weights of both signs, which the
    # magnitude counts in full.
    rng = np.random.default_rng(95 + nd)
    ins = (9, 7, 5)[:nd]
    outs = (4, 6, 3)[:nd]
    data = rng.random((2, 3, *ins)).astype(np.float32)
    nP = int(np.prod(outs))
    gout = rng.standard_normal((2, 3, *outs)).astype(np.float32)
    inside = rng.random((2, nd, nP)).astype(np.float32)
    _, ref = orc.interp_backward(nd, data, inside, outs, np.abs(gout), dtype=np.float64)
    np.testing.assert_allclose(scatter_magnitude(data.shape, inside, outs, gout), ref, rtol=1e-12,
                               atol=1e-12)
    clamped = (rng.random((2, nd, nP)) * 2.0 - 0.5).astype(np.float32)
    _, signed = orc.interp_backward(nd, data, clamped, outs, gout, dtype=np.float64)
    _, plain = orc.interp_backward(nd, data, clamped, outs, np.abs(gout), dtype=np.float64)
    mag = scatter_magnitude(data.shape, clamped, outs, gout)
    assert (np.abs(signed) <= mag + 1e-12).all() and (np.abs(plain) <= mag + 1e-12).all()
    assert (mag > np.abs(plain) + 1e-6).any()


@pytest.mark.parametrize("nd", [2, 3])
def test_interp_matches_torch_grid_sample(nd):
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(91 + nd)
    ins = (11, 8) if nd == 2 else (7, 6, 5)
    outs = (6, 4) if nd == 2 else (4, 3, 5)
    data = rng.random((2, 2, *ins)).astype(np.float32)
    nP = int(np.prod(outs))
    grid = (rng.random((2, nd, nP)) * 1.3 - 0.15).astype(np.float32)
    out = orc.interp_forward(nd, data, grid, outs)
    # grid_sample takes (x, y[, z]) = (last axis, ..., first axis) in [-1, 1]
    g = torch.tensor(grid * 2 - 1)
    pts = g.reshape(2, nd, *outs[::-1])  # [B, nd, o_last, ..., o0] (coordinate 0 fastest)
    pts = pts.flip(1).permute(0, *range(2, 2 + nd), 1)
    ref = F.grid_sample(torch.tensor(data), pts, mode="bilinear", padding_mode="border",
                        align_corners=True)
    ref = ref.permute(0, 1, *range(nd + 1, 1, -1)).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("nd", [1, 2, 3])
def test_interp_backward_matches_finite_differences(nd):
    rng = np.random.default_rng(95 + nd)
    ins = {1: (13,), 2: (9, 8), 3: (6, 5, 7)}[nd]
    outs = {1: (10,), 2: (4, 5), 3: (3, 4, 2)}[nd]
    data = rng.random((2, 2, *ins))
    nP = int(np.prod(outs))
    grid = 0.05 + 0.9 * rng.random((2, nd, nP))
    gout = rng.standard_normal((2, 2, *outs))
    gg, gd = orc.interp_backward(nd, data, grid, outs, gout, dtype=np.float64)
    dg, dd = rng.standard_normal(grid.shape), rng.standard_normal(data.shape)
    eps = 1e-7

    def L(d_, g_):
        return float((gout * orc.interp_forward(nd, d_, g_, outs, dtype=np.float64)).sum())

    fd = (L(data, grid + eps * dg) - L(data, grid - eps * dg)) / (2 * eps)
    assert abs(fd - (gg * dg).sum()) < 1e-6 * max(1, abs(fd))
    fd = (L(data + eps * dd, grid) - L(data - eps * dd, grid)) / (2 * eps)
    assert abs(fd - (gd * dd).sum()) < 1e-6 * max(1, abs(fd))


def test_meshgrid_helper_coordinate0_fastest():
    g = meshgrid([3, 2])
    np.testing.assert_array_equal(g[0], [0, 0.5, 1, 0, 0.5, 1])
    np.testing.assert_array_equal(g[1], [0, 0, 0, 1, 1, 1])
