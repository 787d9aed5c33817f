"""The deterministic backward (``Cpab.set_solver_params(deterministic_grad=True)``,
``cpab_set_deterministic``): two runs give the same moments, theta gradients,
point gradients and transform_data data gradients bit for bit, and each stays
within the oracle's tolerance, as the default mode's float-atomic sums do."""
import numpy as np
import pytest
import torch

from cpab import Cpab
from cpab.pytorch._native import native
from oracle import oracle as orc

from helpers import (assert_adjoint_close, assert_grad_close, assert_theta_grad_close, meshgrid,
                     seeded_theta, uniform_points)

pytestmark = pytest.mark.gpu


def _det_cpab(tess, adaptive=False, nstep=50):
    T = Cpab(list(tess))
    T.set_solver_params(nstepsolver=nstep, adaptive_substeps=adaptive, deterministic_grad=True)
    return T


def _grid_grads(T, theta, pts, g, cuda):
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    x = torch.tensor(pts, device=cuda, requires_grad=True)
    out = T.transform_grid(x, th)
    out.backward(torch.tensor(g, device=cuda))
    return th.grad.cpu().numpy(), x.grad.cpu().numpy()


# [30, 30] and [10, 10, 10] take the LDS cell cache in the integer pass; [20, 20],
# [6, 6] and [3, 3, 3] the row's full table.  nstepsolver 37: the segmented body.
@pytest.mark.parametrize("tess,n,B,adaptive,nstep", [([50], 10000, 4, False, 50),
                                                     ([20, 20], 20000, 4, False, 50),
                                                     ([20, 20], 8000, 2, False, 37),
                                                     ([30, 30], 20000, 3, False, 50),
                                                     ([30, 30], 12000, 3, True, 50),
                                                     ([6, 6], 8000, 2, True, 50),
                                                     ([6, 6], 8000, 2, False, 50),
                                                     ([3, 3, 3], 6000, 2, False, 50),
                                                     ([3, 3, 3], 4000, 2, True, 50),
                                                     ([10, 10, 10], 5000, 2, False, 50),
                                                     ([10, 10, 10], 3000, 2, False, 23)])
def test_transform_grid_repeatable(cuda, tess, n, B, adaptive, nstep):
    T = _det_cpab(tess, adaptive, nstep)
    nd = len(tess)
    theta = seeded_theta(T, B, 0.5, 300 + nd)
    pts = (np.linspace(0, 1, n, dtype=np.float32)[None] if nd == 1 else uniform_points(nd, n, 301))
    g = np.random.default_rng(302).standard_normal((B, nd, n)).astype(np.float32)
    gth1, gx1 = _grid_grads(T, theta, pts, g, cuda)
    gth2, gx2 = _grid_grads(T, theta, pts, g, cuda)
    np.testing.assert_array_equal(gth1, gth2)
    np.testing.assert_array_equal(gx1, gx2)
    assert native().lib.cpab_deterministic() == 0  # the mode does not leak past the backward
    p = T.params
    As = orc.affine(theta, p.basis).reshape(B, p.nC, nd, nd + 1)
    mom, gp = orc.backward(pts, As, g, p.nc, nstep, adaptive=adaptive)
    assert_theta_grad_close(gth1, mom.reshape(B, -1), p.basis)
    assert_adjoint_close(gx1, gp.astype(np.float64).sum(0))


def _moments(cuda, nd, pts, As, g, nc, det, workspace_bytes=None):
    lib = native()
    B, nC = As.shape[0], As.shape[1]
    n = pts.shape[-1]
    x = torch.tensor(pts, device=cuda)
    A = torch.tensor(As, device=cuda)
    go = torch.tensor(g, device=cuda)
    mom = torch.empty((B, nC, nd * (nd + 1)), device=cuda)
    gp = torch.empty((B, nd, n), device=cuda)
    with lib.deterministic(det):
        need = lib.backward_workspace_size(nd, n, B, nC)
        ws = torch.empty(workspace_bytes or need, device=cuda, dtype=torch.uint8)
        lib.backward(nd, x, False, B, n, 50, nc, 0, A, go, mom, gp, ws)
    return mom.cpu().numpy(), gp.cpu().numpy(), need


def test_moments_through_c_abi(cuda):
    # cpab_backward under cpab_set_deterministic: repeatable moments and point
    # adjoints, the oracle's within tolerance, and the mode's own workspace size.
    T = Cpab([20, 20])
    B, n = 3, 30000
    theta = seeded_theta(T, B, 0.6, 310)
    pts = uniform_points(2, n, 311)
    g = np.random.default_rng(312).standard_normal((B, 2, n)).astype(np.float32)
    p = T.params
    As = orc.affine(theta, p.basis).reshape(B, p.nC, 2, 3)
    m1, gp1, need_det = _moments(cuda, 2, pts, As, g, p.nc, True)
    m2, gp2, _ = _moments(cuda, 2, pts, As, g, p.nc, True)
    np.testing.assert_array_equal(m1, m2)
    np.testing.assert_array_equal(gp1, gp2)
    ref_m, ref_gp = orc.backward(pts, As, g, p.nc, 50)
    assert_grad_close(m1.reshape(B, -1), ref_m.reshape(B, -1))
    assert_adjoint_close(gp1, ref_gp)
    m0, _, need_default = _moments(cuda, 2, pts, As, g, p.nc, False)
    assert_grad_close(m0.reshape(B, -1), ref_m.reshape(B, -1))
    # the integer sums and flags take 12 bytes per moment component
    assert need_det >= B * p.nC * 6 * 12
    if need_default < need_det:
        with pytest.raises(RuntimeError, match="workspace too small"):
            _moments(cuda, 2, pts, As, g, p.nc, True, workspace_bytes=need_default)


def test_non_finite_components(cuda):
    # A NaN and an infinite adjoint seed: the components they reach are NaN,
    # +inf or -inf as the default mode's float sums make them, and every
    # other component keeps its finite value.
    T = Cpab([8, 8])
    B, n = 1, 6000
    theta = seeded_theta(T, B, 0.5, 320)
    pts = uniform_points(2, n, 321)
    g = np.random.default_rng(322).standard_normal((B, 2, n)).astype(np.float32)
    g[0, 0, 5] = np.nan
    g[0, 1, 17] = np.inf
    p = T.params
    As = orc.affine(theta, p.basis).reshape(B, p.nC, 2, 3)
    m_det, _, _ = _moments(cuda, 2, pts, As, g, p.nc, True)
    m_def, _, _ = _moments(cuda, 2, pts, As, g, p.nc, False)
    for test in (np.isnan, np.isposinf, np.isneginf):
        np.testing.assert_array_equal(test(m_det), test(m_def))
    assert np.isnan(m_det).any()
    fin = np.isfinite(m_def)
    assert fin.any()
    assert_grad_close(m_det[fin], m_def[fin])


def test_transform_grid_chain_repeatable(cuda):
    T = _det_cpab([16, 16])
    K = 8
    chain = (np.random.default_rng(330).standard_normal((K, T.params.d)) * 0.3).astype(np.float32)
    pts = meshgrid([64, 64])

    def run():
        th = torch.tensor(chain, device=cuda, requires_grad=True)
        x = torch.tensor(pts, device=cuda, requires_grad=True)
        out = T.transform_grid_chain(x, th, scale_by_dt=True)
        g = np.random.default_rng(331).standard_normal(out.shape).astype(np.float32)
        out.backward(torch.tensor(g, device=cuda))
        return th.grad.cpu().numpy(), x.grad.cpu().numpy(), g

    gth, gx, g = run()
    gth2, gx2, _ = run()
    np.testing.assert_array_equal(gth, gth2)
    np.testing.assert_array_equal(gx, gx2)
    p = T.params
    xs, As_all = [pts], []
    for i in range(K):
        As = orc.affine(chain[i:i + 1] * np.float32(1.0 / K), p.basis).reshape(1, p.nC, 2, 3)
        As_all.append(As)
        xs.append(orc.forward_trels(xs[-1], orc.expm(2, As, 1 / 50), As, p.nc, 50))
    lam = g
    for i in reversed(range(K)):
        mom, lam = orc.backward(xs[i], As_all[i], lam, p.nc, 50)
        assert_theta_grad_close(gth[i:i + 1], mom, p.basis, scale=1.0 / K)


@pytest.mark.parametrize("tess,ins", [([30, 30], (64, 48)), ([10, 10, 10], (20, 18, 16))])
def test_transform_data_repeatable(cuda, tess, ins):
    T = _det_cpab(tess)
    nd = len(tess)
    B = 2
    rng = np.random.default_rng(340)
    data = rng.random((B, 1, *ins)).astype(np.float32)
    theta = seeded_theta(T, B, 0.5, 341)
    gout = rng.standard_normal((B, 1, *ins)).astype(np.float32)

    def run():
        th = torch.tensor(theta, device=cuda, requires_grad=True)
        out = T.transform_data(torch.tensor(data, device=cuda), th, list(ins))
        out.backward(torch.tensor(gout, device=cuda))
        return th.grad.cpu().numpy()

    g1, g2 = run(), run()
    np.testing.assert_array_equal(g1, g2)
    p = T.params
    grid = T.uniform_meshgrid(list(ins)).cpu().numpy()  # the start points the kernels take
    As = orc.affine(theta, p.basis).reshape(B, p.nC, nd, nd + 1)
    grid_t = orc.forward_trels(grid, orc.expm(nd, As, 1 / 50), As, p.nc, 50)
    gg, _ = orc.interp_backward(nd, data, grid_t, ins, gout, want_data=False)
    mom, _ = orc.backward(grid, As, gg, p.nc, 50)
    assert_theta_grad_close(g1, mom, p.basis)


@pytest.mark.parametrize("tess,C,ins,outs", [([6, 6], 3, (30, 26), [24, 28]),
                                             ([3, 3, 3], 2, (10, 9, 8), [8, 9, 7]),
                                             ([10], 2, (50,), [40])])
def test_transform_data_data_gradient_repeatable(cuda, tess, C, ins, outs):
    # data and theta both require grad: grad_data, summed as 64-bit integers
    # at each batch row's scale, is the same bit for bit on two runs and within
    # the scatter tolerance of the oracle; the theta gradient too.
    from helpers import scatter_magnitude
    T = _det_cpab(tess)
    nd = len(tess)
    B = 2
    rng = np.random.default_rng(350 + nd)
    data = rng.random((B, C, *ins)).astype(np.float32)
    theta = seeded_theta(T, B, 0.5, 351)
    gout = rng.standard_normal((B, C, *outs)).astype(np.float32)

    def run():
        d_t = torch.tensor(data, device=cuda, requires_grad=True)
        th = torch.tensor(theta, device=cuda, requires_grad=True)
        out = T.transform_data(d_t, th, list(outs))
        out.backward(torch.tensor(gout, device=cuda))
        return d_t.grad.cpu().numpy(), th.grad.cpu().numpy()

    gd1, gth1 = run()
    gd2, gth2 = run()
    np.testing.assert_array_equal(gd1, gd2)
    np.testing.assert_array_equal(gth1, gth2)
    p = T.params
    grid = T.uniform_meshgrid(list(outs)).cpu().numpy()
    As = orc.affine(theta, p.basis).reshape(B, p.nC, nd, nd + 1)
    if nd == 1:
        grid_t = orc.forward_closed_1d(grid, As, p.nc)
    else:
        grid_t = orc.forward_trels(grid, orc.expm(nd, As, 1 / 50), As, p.nc, 50)
    gg, rd = orc.interp_backward(nd, data, grid_t, outs, gout)
    mag = scatter_magnitude(data.shape, grid_t, outs, gout)
    err = np.abs(gd1.astype(np.float64) - rd)
    assert (err <= 1e-4 * mag + 1e-12).all()
    mom, _ = orc.backward(grid, As, gg, p.nc, 50)
    assert_theta_grad_close(gth1, mom, p.basis)


@pytest.mark.parametrize("nd,ins,outs", [(1, (37,), (50,)), (2, (21, 30), (24, 33)),
                                         (3, (9, 8, 10), (7, 6, 9))])
def test_interpolate_data_gradient_repeatable(cuda, nd, ins, outs):
    # Cpab.interpolate under deterministic_grad: the data gradient (summed as
    # 64-bit integers, cpab_interp_backward_ws) is the same on two runs and
    # within the scatter tolerance of the oracle, including points beyond the
    # border (clamped corners, weights outside [0, 1]); grad_grid equals the
    # default path's bit for bit.
    from helpers import scatter_magnitude
    tess = {1: [5], 2: [3, 3], 3: [2, 2, 2]}[nd]
    T = _det_cpab(tess)
    rng = np.random.default_rng(360 + nd)
    B, C = 2, 3
    data = rng.random((B, C, *ins)).astype(np.float32)
    nP = int(np.prod(outs))
    grid = (rng.random((B, nd, nP)) * 1.3 - 0.15).astype(np.float32)
    gout = rng.standard_normal((B, C, *outs)).astype(np.float32)

    def run(params_det):
        T.params.deterministic_grad = params_det
        d_t = torch.tensor(data, device=cuda, requires_grad=True)
        g_t = torch.tensor(grid, device=cuda, requires_grad=True)
        T.interpolate(d_t, g_t, list(outs)).backward(torch.tensor(gout, device=cuda))
        return d_t.grad.cpu().numpy(), g_t.grad.cpu().numpy()

    gd1, gg1 = run(True)
    gd2, gg2 = run(True)
    _, gg0 = run(False)
    T.params.deterministic_grad = True
    np.testing.assert_array_equal(gd1, gd2)
    np.testing.assert_array_equal(gg1, gg2)
    np.testing.assert_array_equal(gg1, gg0)
    _, rd = orc.interp_backward(nd, data, grid, outs, gout)
    mag = scatter_magnitude(data.shape, grid, outs, gout)
    err = np.abs(gd1.astype(np.float64) - rd)
    assert (err <= 1e-4 * mag + 1e-12).all(), float((err / (mag + 1e-30)).max())
