"""Parity at the full sizes of the benchmark configurations (BASELINE.json
configs C1-C5, the inputs bench.py times): each GPU step (forward + gradient)
against the oracle on the same seeded inputs.  Coordinates and images are
held bit-exact; theta-gradients to the 1e-4 relative tolerance.  Kept to the
oracle's speed (a few seconds each on the host's cores)."""
import numpy as np
import pytest
import torch
from scipy.ndimage import gaussian_filter

from oracle import oracle as orc

from helpers import assert_theta_grad_close, cpab_for, seeded_theta

pytestmark = pytest.mark.gpu


def _blur(shape, sigma, seed):
    x = np.random.default_rng(seed).random(shape).astype(np.float32)
    return gaussian_filter(x, sigma=[0, 0] + [sigma] * (len(shape) - 2), mode="reflect",
                           truncate=4.0).astype(np.float32)


def _As(T, theta):
    p = T.params
    return orc.affine(theta, p.basis).reshape(theta.shape[0], p.nC, p.ndim, p.ndim + 1)


def _mse_grad(out, target):
    return ((2.0 / out.size) * (out.astype(np.float64) - target)).astype(np.float32)


@pytest.mark.parametrize("cfg", ["c1", "c2"])
def test_transform_grid_full_size(cuda, cfg):
    if cfg == "c1":
        T = cpab_for([50])
        pts = np.linspace(0, 1, 10_000, dtype=np.float32)[None]
        theta, theta_t = seeded_theta(T, 16, 0.5, 11), seeded_theta(T, 16, 0.5, 12)
    else:
        T = cpab_for([20, 20])
        pts = np.random.default_rng(21).random((2, 125_000)).astype(np.float32)
        theta, theta_t = seeded_theta(T, 16, 0.5, 22), seeded_theta(T, 16, 0.5, 23)
    p = T.params
    nd = p.ndim
    x = torch.tensor(pts, device=cuda)
    with torch.no_grad():
        target = T.transform_grid(x, torch.tensor(theta_t, device=cuda))
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    out = T.transform_grid(x, th)
    torch.mean((out - target) ** 2).backward()

    As = _As(T, theta)
    if nd == 1:
        ref = orc.forward_closed_1d(pts, As, p.nc)
    else:
        ref = orc.forward_trels(pts, orc.expm(nd, As, 1 / 50), As, p.nc, 50)
    out_np = out.detach().cpu().numpy()
    np.testing.assert_array_equal(out_np, ref)
    g = _mse_grad(out_np, target.cpu().numpy())
    mom, _ = orc.backward(pts, As, g, p.nc, 50)
    assert_theta_grad_close(th.grad.cpu().numpy(), mom, p.basis)


@pytest.mark.parametrize("cfg", ["c3", "c4"])
def test_transform_data_full_size(cuda, cfg):
    if cfg == "c3":
        T, B, size, sigma, seeds = cpab_for([30, 30]), 16, [512, 512], 4.0, (31, 32, 33)
    else:
        T, B, size, sigma, seeds = cpab_for([10, 10, 10]), 1, [128, 128, 128], 3.0, (41, 42, 43)
    p = T.params
    nd = p.ndim
    data = _blur((B, 1, *size), sigma, seeds[0])
    target = _blur((B, 1, *size), sigma, seeds[1])
    theta = seeded_theta(T, B, 0.5, seeds[2])
    th = torch.tensor(theta, device=cuda, requires_grad=True)
    out = T.transform_data(torch.tensor(data, device=cuda), th, size)
    torch.mean((out - torch.tensor(target, device=cuda)) ** 2).backward()

    grid = T.uniform_meshgrid(size).cpu().numpy()
    As = _As(T, theta)
    grid_t = orc.forward_trels(grid, orc.expm(nd, As, 1 / 50), As, p.nc, 50)
    ref = orc.interp_forward(nd, data, grid_t, size)
    out_np = out.detach().cpu().numpy()
    np.testing.assert_array_equal(out_np, ref)
    gimg = _mse_grad(out_np, target)
    gg, _ = orc.interp_backward(nd, data, grid_t, size, gimg, want_data=False)
    mom, _ = orc.backward(grid, As, gg, p.nc, 50)
    assert_theta_grad_close(th.grad.cpu().numpy(), mom, p.basis)


def test_transform_grid_chain_full_size(cuda):
    T = cpab_for([16, 16])
    p = T.params
    K = 8
    chain = (np.random.default_rng(51).standard_normal((K, p.d)) * 0.3).astype(np.float32)
    chain_t = (np.random.default_rng(52).standard_normal((K, p.d)) * 0.3).astype(np.float32)
    grid_t = T.uniform_meshgrid([512, 512])
    with torch.no_grad():
        target = T.transform_grid_chain(grid_t, torch.tensor(chain_t, device=cuda), scale_by_dt=True)
    ch = torch.tensor(chain, device=cuda, requires_grad=True)
    out = T.transform_grid_chain(grid_t, ch, scale_by_dt=True)
    torch.mean((out - target) ** 2).backward()

    xs = [grid_t.cpu().numpy()]
    As_all = []
    for i in range(K):
        th_i = chain[i:i + 1] * np.float32(1.0 / K)
        As = _As(T, th_i)
        As_all.append(As)
        xs.append(orc.forward_trels(xs[-1], orc.expm(2, As, 1 / 50), As, p.nc, 50))
    out_np = out.detach().cpu().numpy()
    np.testing.assert_array_equal(out_np, xs[-1])
    lam = _mse_grad(out_np, target.cpu().numpy())
    gch = ch.grad.cpu().numpy()
    for i in reversed(range(K)):
        mom, lam = orc.backward(xs[i], As_all[i], lam, p.nc, 50)
        assert_theta_grad_close(gch[i:i + 1], mom, p.basis, scale=1.0 / K)
