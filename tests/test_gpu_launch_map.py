"""The backward's own workgroup map (wg_slot in backward_body.hpp), exercised on the
GPU: grids whose workgroup count is not a multiple of the 8 XCDs, row counts
that leave a partial block of rows, one theta row, and the segmented variant's
other launch shape.  Outputs are prefilled with NaN, so a (point range, theta
row) that no workgroup took leaves NaN behind, and one taken twice doubles its
moments; both are checked against the oracle.  (tests/test_launch_maps.py
checks the same map's arithmetic on the CPU for every grid up to 40 x 20.)"""
import numpy as np
import pytest
import torch

from cpab.pytorch._native import native
from cpab.pytorch.transformer import basis_tables
from oracle import oracle as orc

from helpers import assert_adjoint_close, assert_grad_close, cpab_for, seeded_theta, uniform_points

pytestmark = pytest.mark.gpu


# (n_theta, nP, nstepsolver): at T = 50 the register variant takes ~256 workgroups
# of 1024 lanes (3 x 86, 5 x 52, 7 x 37, 13 x 20, 1 x 256); T = 37 the segmented one.
@pytest.mark.parametrize("n_theta,nP,T", [(3, 90000, 50), (5, 60000, 50), (7, 40000, 50),
                                          (13, 25000, 50), (1, 300000, 50), (6, 30000, 37)])
def test_every_range_and_row_taken_once(cuda, n_theta, nP, T):
    Tc = cpab_for([20, 20])
    p = Tc.params
    theta = seeded_theta(Tc, n_theta, 0.5, 400 + n_theta)
    pts = uniform_points(2, nP, 401)
    g = np.random.default_rng(402).standard_normal((n_theta, 2, nP)).astype(np.float32)
    As = orc.affine(theta, p.basis).reshape(n_theta, p.nC, 2, 3)
    lib = native()
    mom = torch.full((n_theta, p.nC, 6), float("nan"), device=cuda)
    gp = torch.full((n_theta, 2, nP), float("nan"), device=cuda)
    ws = torch.empty(lib.backward_workspace_size(2, nP, n_theta, p.nC), dtype=torch.uint8,
                     device=cuda)
    lib.backward(2, torch.tensor(pts, device=cuda), False, n_theta, nP, T, p.nc, 0,
                 torch.tensor(As, device=cuda), torch.tensor(g, device=cuda), mom, gp, ws)
    mom, gp = mom.cpu().numpy(), gp.cpu().numpy()
    assert np.isfinite(gp).all() and np.isfinite(mom).all()
    ref_m, ref_gp = orc.backward(pts, As, g, p.nc, T)
    assert_grad_close(mom.reshape(n_theta, -1), ref_m.reshape(n_theta, -1))
    assert_adjoint_close(gp, ref_gp)
