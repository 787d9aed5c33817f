"""End-to-end parity of the drop-in ``Cpab`` API on the GPU against the oracle:
transform_grid forward + autograd backward (theta and points), transform_data,
transform_grid_chain, on the benchmark configurations at reduced sizes."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

from helpers import (assert_theta_grad_close, cpab_for, meshgrid, scatter_magnitude, seeded_theta,
                     uniform_points)

pytestmark = pytest.mark.gpu


def _oracle_grid(T, theta, pts, g_out, nstep=50):
    """Oracle forward, moments [n_theta, D] (theta gradient B^T m) and points
    gradient of <out, g_out>."""
    p = T.params
    nd = p.ndim
    As = orc.affine(theta, p.basis).reshape(theta.shape[0], p.nC, nd, nd + 1)
    if nd == 1:
        out = orc.forward_closed_1d(pts, As, p.nc)
    else:
        out = orc.forward_trels(pts, orc.expm(nd, As, 1.0 / nstep), As, p.nc, nstep)
    mom, gp = orc.backward(pts, As, g_out, p.nc, nstep)
    if pts.ndim == 2:
        gp = gp.astype(np.float64).sum(0)
    return out, mom.reshape(theta.shape[0], -1), gp


@pytest.mark.parametrize("tess,n,B", [([50], 10000, 16), ([20, 20], 20000, 4),
                                      ([16, 16], 30000, 2), ([10, 10, 10], 5000, 2)])
def test_transform_grid_fwd_bwd(cuda, tess, n, B):
    T = cpab_for(tess)
    nd = len(tess)
    theta = seeded_theta(T, B, 0.5, 200 + nd)
    pts = (np.linspace(0, 1, n, dtype=np.float32)[None] if nd == 1 else uniform_points(nd, n, 201))
    g = np.random.default_rng(202).standard_normal((B, nd, n)).astype(np.float32)
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    x = torch.tensor(pts, device=cuda, requires_grad=True)
    out = T.transform_grid(x, th)
    out.backward(torch.tensor(g, device=cuda))
    ref_out, ref_m, ref_gp = _oracle_grid(T, theta, pts, g)
    np.testing.assert_allclose(out.detach().cpu().numpy(), ref_out, atol=1e-5, rtol=0)
    assert_theta_grad_close(th.grad.cpu().numpy(), ref_m, T.params.basis)
    np.testing.assert_allclose(x.grad.cpu().numpy(), ref_gp, rtol=1e-5,
                               atol=1e-6 * np.abs(ref_gp).max())


def test_retained_graph_backward_twice(cuda):
    # A retained graph's backward runs twice on the same saved tensors (the
    # forward's As and points): both give the oracle's gradient, and the
    # points' gradient is the same bit for bit.
    T = cpab_for([20, 20])
    theta = seeded_theta(T, 4, 0.5, 230)
    pts = uniform_points(2, 20000, 231)
    g = np.random.default_rng(232).standard_normal((4, 2, 20000)).astype(np.float32)
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    x = torch.tensor(pts, device=cuda, requires_grad=True)
    out = T.transform_grid(x, th)
    gt = torch.tensor(g, device=cuda)
    out.backward(gt, retain_graph=True)
    g1, x1 = th.grad.clone(), x.grad.clone()
    th.grad, x.grad = None, None
    out.backward(gt)
    _, ref_m, _ = _oracle_grid(T, theta, pts, g)
    for gth in (g1, th.grad):
        assert_theta_grad_close(gth.cpu().numpy(), ref_m, T.params.basis)
    np.testing.assert_array_equal(x1.cpu().numpy(), x.grad.cpu().numpy())


def test_transform_grid_mse_loss_c2_shape(cuda):
    # C2's loss: MSE to a second seeded theta's warped points (reduced nP).
    T = cpab_for([20, 20])
    pts = uniform_points(2, 25000, 21)
    theta = seeded_theta(T, 16, 0.5, 22)
    theta_t = seeded_theta(T, 16, 0.5, 23)
    x = torch.tensor(pts, device=cuda)
    with torch.no_grad():
        target = T.transform_grid(x, torch.tensor(theta_t, device=cuda))
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    out = T.transform_grid(x, th)
    loss = ((out - target) ** 2).mean()
    loss.backward()
    g = (2.0 / out.numel()) * (out - target).detach().cpu().numpy().astype(np.float32)
    ref_out, ref_m, _ = _oracle_grid(T, theta, pts, g)
    np.testing.assert_allclose(out.detach().cpu().numpy(), ref_out, atol=1e-5, rtol=0)
    assert_theta_grad_close(th.grad.cpu().numpy(), ref_m, T.params.basis)


@pytest.mark.parametrize("tess,ins", [([30, 30], (64, 48)), ([10, 10, 10], (20, 18, 16))])
def test_transform_data(cuda, tess, ins):
    T = cpab_for(tess)
    nd = len(tess)
    B = 2
    rng = np.random.default_rng(31)
    data = rng.random((B, 1, *ins)).astype(np.float32)
    theta = seeded_theta(T, B, 0.5, 33)
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    out = T.transform_data(torch.tensor(data, device=cuda), th, list(ins))
    gout = rng.standard_normal(out.shape).astype(np.float32)
    out.backward(torch.tensor(gout, device=cuda))
    grid = T.uniform_meshgrid(list(ins)).cpu().numpy()
    # torch's device linspace may differ from numpy's by an ulp
    np.testing.assert_allclose(grid, meshgrid(list(ins)), rtol=0, atol=1.2e-7)
    p = T.params
    As = orc.affine(theta, p.basis).reshape(B, p.nC, nd, nd + 1)
    grid_t = orc.forward_trels(grid, orc.expm(nd, As, 1 / 50), As, p.nc, 50)
    ref = orc.interp_forward(nd, data, grid_t, ins)
    np.testing.assert_allclose(out.detach().cpu().numpy(), ref, atol=1e-5, rtol=0)
    gg, _ = orc.interp_backward(nd, data, grid_t, ins, gout, want_data=False)
    mom, _ = orc.backward(grid, As, gg, p.nc, 50)
    assert_theta_grad_close(th.grad.cpu().numpy(), mom, p.basis)


def test_transform_data_data_gradient(cuda):
    # data and theta both require grad (e.g. a learned template image): the
    # fused backward returns both.
    T = cpab_for([6, 6])
    B, C, ins, outs = 2, 3, (30, 26), [24, 28]
    rng = np.random.default_rng(35)
    data = rng.random((B, C, *ins)).astype(np.float32)
    theta = seeded_theta(T, B, 0.5, 36)
    d_t = torch.tensor(data, device=cuda, requires_grad=True)
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    out = T.transform_data(d_t, th, outs)
    gout = rng.standard_normal(out.shape).astype(np.float32)
    out.backward(torch.tensor(gout, device=cuda))
    grid = T.uniform_meshgrid(outs).cpu().numpy()
    p = T.params
    As = orc.affine(theta, p.basis).reshape(B, p.nC, 2, 3)
    grid_t = orc.forward_trels(grid, orc.expm(2, As, 1 / 50), As, p.nc, 50)
    _, rd = orc.interp_backward(2, data, grid_t, outs, gout)
    mag = scatter_magnitude(data.shape, grid_t, outs, gout)
    err = np.abs(d_t.grad.cpu().numpy().astype(np.float64) - rd)
    assert (err <= 1e-4 * mag + 1e-12).all()
    assert th.grad is not None and torch.isfinite(th.grad).all()
    # theta only (data without grad) and no grad at all also run
    out2 = T.transform_data(torch.tensor(data, device=cuda), th.detach(), outs)
    np.testing.assert_array_equal(out2.cpu().numpy(), out.detach().cpu().numpy())


def test_transform_grid_chain(cuda):
    T = cpab_for([16, 16])
    K = 8
    chain = (np.random.default_rng(51).standard_normal((K, T.params.d)) * 0.3).astype(np.float32)
    pts = meshgrid([64, 64])
    th = torch.tensor(chain, device=cuda, requires_grad=True)
    out = T.transform_grid_chain(torch.tensor(pts, device=cuda), th, scale_by_dt=True)
    g = np.random.default_rng(52).standard_normal(out.shape).astype(np.float32)
    out.backward(torch.tensor(g, device=cuda))
    # Oracle: K stages forward, then reverse-mode through the stages.
    p = T.params
    xs = [pts]
    As_all = []
    for i in range(K):
        th_i = chain[i:i + 1] * np.float32(1.0 / K)
        As = orc.affine(th_i, p.basis).reshape(1, p.nC, 2, 3)
        As_all.append(As)
        xs.append(orc.forward_trels(xs[-1], orc.expm(2, As, 1 / 50), As, p.nc, 50))
    np.testing.assert_allclose(out.detach().cpu().numpy(), xs[-1], atol=1e-5, rtol=0)
    lam = g
    gth = th.grad.cpu().numpy()
    for i in reversed(range(K)):
        mom, gp = orc.backward(xs[i], As_all[i], lam, p.nc, 50)
        assert_theta_grad_close(gth[i:i + 1], mom, p.basis, scale=1.0 / K)
        lam = gp


def _corner_heavy_points(nd, n, seed):
    """Uniform points in [0,1]^nd, a quarter of them within 0.06 of a corner
    (where fields that are not zero on the boundary carry trajectories past
    the domain's corners and the out-of-domain lookup rules decide the cell)."""
    rng = np.random.default_rng(seed)
    pts = rng.random((nd, n))
    k = n // 4
    corner = rng.integers(0, 2, (nd, k)).astype(np.float64)
    pts[:, :k] = np.abs(corner - 0.06 * rng.random((nd, k)))
    return pts.astype(np.float32)


@pytest.mark.parametrize("tess,zb,vp,scale,n", [([20, 20], False, False, 1.0, 20000),
                                                ([4, 4, 3], False, False, 1.0, 8000),
                                                ([7], False, False, 1.0, 5000),
                                                ([6, 5], True, True, 1.0, 8000),
                                                ([20, 20], False, True, 1.0, 8000),
                                                ([3, 3, 3], False, True, 1.0, 6000),
                                                # strong: checkpoint replay in the backward
                                                ([4, 4, 3], False, False, 4.0, 6000)])
def test_general_basis_end_to_end(cuda, tess, zb, vp, scale, n):
    # Bases from the SVD null space (zero_boundary=False, volume_perservation):
    # fields that move points across the domain boundary, so the forward, the
    # replay and the adjoint run through the out-of-domain cell rules
    # (cpab_ops_2d.cu:97-117, the 3D corner rule cpab_ops_3d.cu:79-88) on
    # the outside-continuity constraints of tesselation.py:392-429,515-544.
    from cpab import Cpab
    T = Cpab(tess, zero_boundary=zb, volume_perservation=vp)
    nd = len(tess)
    B = 2
    theta = seeded_theta(T, B, scale, 210 + nd)
    pts = (_corner_heavy_points(nd, n, 211) if nd > 1
           else np.linspace(0, 1, n, dtype=np.float32)[None])
    g = np.random.default_rng(212).standard_normal((B, nd, n)).astype(np.float32)
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    x = torch.tensor(pts, device=cuda, requires_grad=True)
    out = T.transform_grid(x, th)
    out.backward(torch.tensor(g, device=cuda))
    res = out.detach().cpu().numpy()
    outside = ((res < 0) | (res > 1)).any(axis=1)
    if not zb:
        assert outside.mean() > 0.01, outside.mean()
        if nd == 3 and not vp:  # some trajectories end beyond a corner of the cube
            assert ((res < 0) | (res > 1)).all(axis=1).sum() > 10
    ref_out, ref_m, ref_gp = _oracle_grid(T, theta, pts, g)
    np.testing.assert_allclose(res, ref_out, atol=1e-5, rtol=0)
    assert_theta_grad_close(th.grad.cpu().numpy(), ref_m, T.params.basis)
    np.testing.assert_allclose(x.grad.cpu().numpy(), ref_gp, rtol=1e-5,
                               atol=1e-6 * np.abs(ref_gp).max())


def test_identity_theta_is_identity(cuda):
    for tess in ([50], [20, 20], [10, 10, 10]):
        T = cpab_for(tess)
        nd = len(tess)
        pts = uniform_points(nd, 4000, 7)
        out = T.transform_grid(torch.tensor(pts, device=cuda), T.identity(3))
        np.testing.assert_array_equal(out.cpu().numpy(), np.broadcast_to(pts, (3, nd, 4000)))


def test_stn_cpabwarp_style_composition(cuda):
    # stn/stn.py:68-86 (CpabWarp.transform) calls the drop-in exactly like this:
    # pixel grid in [-1, 1] flipped to CPAB order, then
    # CPAB_transformer(points, theta, params, points.requires_grad) for each warp
    # of a composition, the last warp first.  Check the composed output and both
    # thetas' gradients against the oracle's stage-by-stage reverse mode.
    from cpab.pytorch.transformer import CPAB_transformer
    T = cpab_for([4, 5])
    p = T.params
    B, H, W = 2, 20, 24
    ys, xs = torch.linspace(-1, 1, H, device=cuda), torch.linspace(-1, 1, W, device=cuda)
    pix = torch.stack(torch.meshgrid(ys, xs, indexing="ij")[::-1]).flatten(1)  # [2, P] (x, y)
    th1 = torch.tensor(seeded_theta(T, B, 0.4, 41), device=cuda, requires_grad=True)
    th2 = torch.tensor(seeded_theta(T, B, 0.4, 42), device=cuda, requires_grad=True)
    pts = (pix.flip(-2) + 1) / 2
    for th in (th2, th1):  # T_K acts first
        pts = CPAB_transformer(pts, th, p, pts.requires_grad)
    out = (pts * 2 - 1).flip(-2)
    g = np.random.default_rng(43).standard_normal(out.shape).astype(np.float32)
    out.backward(torch.tensor(g, device=cuda))

    x0 = ((pix.flip(-2) + 1) / 2).cpu().numpy()
    A2 = orc.affine(th2.detach().cpu().numpy(), p.basis).reshape(B, p.nC, 2, 3)
    A1 = orc.affine(th1.detach().cpu().numpy(), p.basis).reshape(B, p.nC, 2, 3)
    x1 = orc.forward_trels(x0, orc.expm(2, A2, 1 / 50), A2, p.nc, 50)
    x2 = orc.forward_trels(x1, orc.expm(2, A1, 1 / 50), A1, p.nc, 50)
    np.testing.assert_allclose(out.detach().cpu().numpy(), (x2 * 2 - 1)[:, ::-1], atol=2e-6, rtol=0)
    lam = (2 * g[:, ::-1]).astype(np.float32)  # d out / d x2 through the flip and scale
    m1, lam1 = orc.backward(x1, A1, lam, p.nc, 50)
    m2, _ = orc.backward(x0, A2, lam1, p.nc, 50)
    assert_theta_grad_close(th1.grad.cpu().numpy(), m1, p.basis)
    assert_theta_grad_close(th2.grad.cpu().numpy(), m2, p.basis)


def test_runs_on_current_stream(cuda):
    # Kernels are enqueued on torch's current stream: results computed inside a
    # side stream (default priority) match the default stream's.
    T = cpab_for([8, 8])
    pts = torch.tensor(uniform_points(2, 5000, 51), device=cuda)
    th = torch.tensor(seeded_theta(T, 3, 0.5, 52), device=cuda)
    ref = T.transform_grid(pts, th)
    side = torch.cuda.Stream(device=cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        out = T.transform_grid(pts, th)
    side.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
