"""The reference-side binding (cpab/pytorch/cpab_gpu_hip.py), called the way the
reference's _CPABFunction calls its cpab_gpu module
(cpab/pytorch/transformer.py:72-168): A = torch.sparse.mm(B, theta^T), then
expm on the flat [n_theta * nC, ndim, ndim+1] blocks and forward (2D/3D), or
forward_1d_closed_form (1D); backward_moments[_and_points] with the saved
points and As, then the projection.  Checked against the oracle on the same As:
forward bit for bit, moments and point adjoints within the backward's
tolerance.  3D tessellations have ncz different from ncx and ncy, so the
binding's ncz inference (transformer_cuda.cu:65-75) decides the result."""
import numpy as np
import pytest
import torch

from cpab.pytorch import cpab_gpu_hip as cpab_gpu
from oracle import oracle as orc

from helpers import (assert_adjoint_close, assert_grad_close, assert_theta_grad_close, cpab_for,
                     seeded_theta, uniform_points)

pytestmark = pytest.mark.gpu


def _reference_forward(T, theta, points, adaptive, cuda):
    """_CPABFunction.forward of the reference (transformer.py:72-126) on cpab_gpu_hip."""
    p = T.params
    B = p.basis.tocoo()
    B_sparse = torch.sparse_coo_tensor(np.vstack([B.row, B.col]), B.data.astype(np.float32),
                                       B.shape, device=cuda).coalesce()
    th = torch.tensor(theta, device=cuda)
    n_theta = th.shape[0]
    Avees = torch.sparse.mm(B_sparse, th.t())
    As = Avees.t().reshape(n_theta * p.nC, p.ndim, p.ndim + 1)
    As_batch = As.view(n_theta, p.nC, p.ndim, p.ndim + 1)
    ncx = int(p.nc[0])
    ncy = int(p.nc[1]) if p.ndim > 1 else 1
    if p.ndim == 1:
        out = cpab_gpu.forward_1d_closed_form(points.contiguous(), As_batch.contiguous(), ncx)
        Trels = None
    else:
        Trels = cpab_gpu.expm(As.contiguous(), 1.0 / p.nstepsolver)
        Trels = Trels.view(n_theta, p.nC, p.ndim, p.ndim + 1)
        out = cpab_gpu.forward(points.contiguous(), Trels.contiguous(), As_batch.contiguous(),
                               p.nstepsolver, ncx, ncy, adaptive)
    return As_batch, Trels, out, ncx, ncy


@pytest.mark.parametrize("tess,batched,adaptive", [([12], False, 0), ([12], True, 0),
                                                   ([8, 6], False, 0), ([8, 6], True, 1),
                                                   ([3, 2, 4], False, 0), ([3, 2, 4], True, 0)])
def test_binding_like_cpabfunction(cuda, tess, batched, adaptive):
    T = cpab_for(tess)
    p = T.params
    nd = p.ndim
    n_theta, nP = 3, 4000
    theta = seeded_theta(T, n_theta, 0.5, 240 + nd)
    pts_np = (np.random.default_rng(241).random((n_theta, nd, nP)).astype(np.float32) if batched
              else uniform_points(nd, nP, 241))
    points = torch.tensor(pts_np, device=cuda)
    As_batch, Trels, out, ncx, ncy = _reference_forward(T, theta, points, adaptive, cuda)
    A = As_batch.cpu().numpy()
    if nd == 1:
        ref = orc.forward_closed_1d(pts_np, A, p.nc)
        # the generic forward dispatches 1D to the same closed form
        np.testing.assert_array_equal(
            cpab_gpu.forward(points, As_batch.contiguous(), As_batch.contiguous(), 50, ncx, 1, 0)
            .cpu().numpy(), ref)
    else:
        Tr = orc.expm(nd, A, 1.0 / 50)
        np.testing.assert_array_equal(Trels.cpu().numpy(), Tr)
        ref = orc.forward_trels(pts_np, Tr, A, p.nc, 50, adaptive=bool(adaptive))
    np.testing.assert_array_equal(out.cpu().numpy(), ref)

    g = np.random.default_rng(242).standard_normal((n_theta, nd, nP)).astype(np.float32)
    grad = torch.tensor(g, device=cuda)
    moments, grad_points = cpab_gpu.backward_moments_and_points(points, As_batch.contiguous(), grad,
                                                                50, ncx, ncy, adaptive)
    ref_m, ref_gp = orc.backward(pts_np, A, g, p.nc, 50, adaptive=bool(adaptive))
    assert tuple(moments.shape) == (n_theta, p.nC, nd * (nd + 1))
    assert tuple(grad_points.shape) == (n_theta, nd, nP)
    assert_grad_close(moments.cpu().numpy(), ref_m, rtol=2e-5)
    assert_adjoint_close(grad_points.cpu().numpy(), ref_gp)
    m_only = cpab_gpu.backward_moments(points, As_batch.contiguous(), grad, 50, ncx, ncy, adaptive)
    assert_grad_close(m_only.cpu().numpy(), ref_m, rtol=2e-5)
    # transformer.py:165-166: the projection onto the basis
    Bt = p.basis.T.tocoo()
    Bt_sparse = torch.sparse_coo_tensor(np.vstack([Bt.row, Bt.col]), Bt.data.astype(np.float32),
                                        Bt.shape, device=cuda).coalesce()
    grad_theta = torch.sparse.mm(Bt_sparse, moments.reshape(n_theta, -1).t()).t()
    assert_theta_grad_close(grad_theta.cpu().numpy(), ref_m, p.basis)


def test_binding_expm_1d_and_3d_shapes(cuda):
    # expm takes [n, ndim, ndim+1]; the 1D form ([n, 1, 2]) is reachable only
    # through the binding (the reference's 1D path never calls it).
    for nd in (1, 2, 3):
        A = (np.random.default_rng(250 + nd).standard_normal((37, nd, nd + 1)) * 2.0).astype(np.float32)
        out = cpab_gpu.expm(torch.tensor(A, device=cuda), 0.3)
        np.testing.assert_array_equal(out.cpu().numpy(), orc.expm(nd, A, 0.3))


def test_binding_errors(cuda):
    T = cpab_for([3, 2, 4])
    p = T.params
    As = torch.zeros((1, p.nC - 5, 3, 4), device=cuda)    # nC not a multiple of 5*ncx*ncy
    pts = torch.rand((3, 100), device=cuda)
    g = torch.zeros((1, 3, 100), device=cuda)
    with pytest.raises(RuntimeError, match="Could not infer ncz"):
        cpab_gpu.backward_moments(pts, As, g, 50, 3, 2, 0)
    with pytest.raises(RuntimeError, match="adaptive_substeps"):
        cpab_gpu.backward_moments(pts, torch.zeros((1, p.nC, 3, 4), device=cuda), g, 50, 3, 2, 2)
    with pytest.raises(RuntimeError, match="CPAB_MAX_STEPS"):
        cpab_gpu.backward_moments(pts, torch.zeros((1, p.nC, 3, 4), device=cuda), g, 101, 3, 2, 0)
    with pytest.raises(RuntimeError, match="contiguous float32"):
        cpab_gpu.expm(torch.zeros((4, 2, 3), device=cuda, dtype=torch.float64), 0.1)
    with pytest.raises(RuntimeError, match="shape"):
        cpab_gpu.forward_1d_closed_form(torch.rand((1, 10), device=cuda),
                                        torch.zeros((1, 4, 2, 3), device=cuda), 4)
