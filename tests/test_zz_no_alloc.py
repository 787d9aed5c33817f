"""cpab_backward_noalloc (the allocation-free backward, through the C ABI)
against cpab_backward with a caller workspace: same kernels, so moments and
point adjoints agree to the summation-order tolerance of the moment sums (the
float atomics add in no fixed order).  Two calls in a row, the second smaller,
then a third of another dimension: the library's per-GPU scratch keeps the
last call's contents, so each call must clear what it accumulates into."""
import ctypes

import numpy as np
import pytest
import torch

from cpab.pytorch._native import native
from cpab.pytorch.transformer import basis_tables

from helpers import assert_adjoint_close, assert_grad_close, cpab_for, seeded_theta, uniform_points

pytestmark = pytest.mark.gpu


def _dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _case(cuda, tess, n_theta, nP, batched, seed, scale=0.5):
    T = cpab_for(tess)
    p = T.params
    nd = len(tess)
    theta = seeded_theta(T, n_theta, scale, seed)
    tab = basis_tables(p, cuda)
    As = torch.empty((n_theta, p.nC, nd, nd + 1), device=cuda)
    native().affine(nd, _dev(theta, cuda), p.nC, tab["row_ptr"], tab["col_idx"], tab["vals"], As)
    if batched:
        pts = np.random.default_rng(seed + 1).random((n_theta, nd, nP)).astype(np.float32)
    else:
        pts = uniform_points(nd, nP, seed + 1)
    g = np.random.default_rng(seed + 2).standard_normal((n_theta, nd, nP)).astype(np.float32)
    return p, _dev(pts, cuda), As, _dev(g, cuda)


def _both(cuda, p, pts, As, g, batched, nstep=50, adaptive=0):
    nd = p.ndim
    n_theta, nP = As.shape[0], pts.shape[-1]
    ppc = nd * (nd + 1)
    ref_m = torch.empty((n_theta, p.nC, ppc), device=cuda)
    ref_gp = torch.empty((n_theta, nd, nP), device=cuda)
    nbytes = native().backward_workspace_size(nd, nP, n_theta, p.nC)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    native().backward(nd, pts, batched, n_theta, nP, nstep, p.nc, adaptive, As, g, ref_m, ref_gp, ws)
    # outputs prefilled with garbage: the entry point overwrites them
    m = torch.full((n_theta, p.nC, ppc), 7.0, device=cuda)
    gp = torch.full((n_theta, nd, nP), -3.0, device=cuda)
    native().backward_noalloc(nd, pts, batched, n_theta, nP, nstep, p.nc, adaptive, As, g, m, gp)
    torch.cuda.synchronize()
    assert_grad_close(m.cpu().numpy(), ref_m.cpu().numpy(), rtol=2e-5)
    assert_adjoint_close(gp.cpu().numpy(), ref_gp.cpu().numpy())


def test_noalloc_matches_workspace_backward(cuda):
    # first call: C2-like (full LDS bins, dense partial tables in the scratch)
    p, pts, As, g = _case(cuda, [20, 20], 8, 20000, False, 301)
    _both(cuda, p, pts, As, g, False)
    torch.cuda.synchronize()
    free_after_setup = torch.cuda.mem_get_info()[0]
    # second call, smaller: fewer cells, thetas and points, batched points
    p, pts, As, g = _case(cuda, [4, 4], 2, 300, True, 302)
    _both(cuda, p, pts, As, g, True)
    # third: 3D, then the segmented variant (nstepsolver != 50)
    p, pts, As, g = _case(cuda, [4, 4, 4], 3, 4000, False, 303)
    _both(cuda, p, pts, As, g, False)
    p, pts, As, g = _case(cuda, [20, 20], 2, 3000, False, 304)
    _both(cuda, p, pts, As, g, False, nstep=37)
    torch.cuda.synchronize()
    # nothing was allocated on the device by the calls after the first
    # (torch's own allocations above are freed back into its cache)
    assert torch.cuda.mem_get_info()[0] >= free_after_setup


def test_noalloc_rejects_beyond_limit(cuda):
    # 1000 thetas x 1600 cells: the reverse-sweep table alone is 77 MB, beyond
    # the 32 MiB scratch; rejected before anything is enqueued
    p, pts, As, g = _case(cuda, [20, 20], 1000, 10, False, 305)
    m = torch.empty((1000, p.nC, 6), device=cuda)
    lib = native().lib
    rc = lib.cpab_backward_noalloc(2, 10, 1000, 0, 50, 20, 20, 1, 0, ctypes.c_void_p(pts.data_ptr()),
                                   ctypes.c_void_p(As.data_ptr()), ctypes.c_void_p(g.data_ptr()),
                                   ctypes.c_void_p(m.data_ptr()), None, None)
    assert rc == 1
    msg = lib.cpab_last_error_string().decode()
    assert "no-allocation limit" in msg, msg
    # and a problem that fits still runs after the rejection
    p, pts, As, g = _case(cuda, [4, 4], 2, 500, False, 306)
    _both(cuda, p, pts, As, g, False)


def test_noalloc_under_graph_capture(cuda):
    # The callers the entry point is for include code under HIP graph capture:
    # record it into a torch CUDA graph in global capture mode (an allocation,
    # a synchronisation or another capture-unsafe call in any thread then
    # fails the capture), replay it with the inputs changed in place and eager
    # work and synchronisations between the replays, and check every replay
    # against cpab_backward with a workspace.  Every tensor is allocated before
    # the capture, and the first (eager) call sets up the scratch address and
    # kernel attributes outside it.
    p, pts, As, g = _case(cuda, [20, 20], 4, 8000, False, 307)
    nd, ppc = p.ndim, p.ndim * (p.ndim + 1)
    n_theta, nP = As.shape[0], pts.shape[-1]
    g0 = g.clone()
    ref_m = torch.empty((n_theta, p.nC, ppc), device=cuda)
    ref_gp = torch.empty((n_theta, nd, nP), device=cuda)
    ws = torch.empty(native().backward_workspace_size(nd, nP, n_theta, p.nC), dtype=torch.uint8,
                     device=cuda)
    native().backward(nd, pts, False, n_theta, nP, 50, p.nc, 0, As, g0, ref_m, ref_gp, ws)
    m = torch.empty((n_theta, p.nC, ppc), device=cuda)
    gp = torch.empty((n_theta, nd, nP), device=cuda)
    native().backward_noalloc(nd, pts, False, n_theta, nP, 50, p.nc, 0, As, g, m, gp)
    torch.cuda.synchronize()
    assert_grad_close(m.cpu().numpy(), ref_m.cpu().numpy(), rtol=2e-5)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="global"):
        native().backward_noalloc(nd, pts, False, n_theta, nP, 50, p.nc, 0, As, g, m, gp)
    torch.cuda.synchronize()
    ref_m, ref_gp = ref_m.cpu().numpy(), ref_gp.cpu().numpy()
    for k in (1.0, 2.0, 0.5, 1.0):
        # the backward is linear in grad_out, and scaling by a power of two is
        # exact: the replay must follow the new input
        g.copy_(g0 * k)
        m.fill_(7.0)
        gp.fill_(-3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_grad_close(m.cpu().numpy(), ref_m * k, rtol=2e-5)
        assert_adjoint_close(gp.cpu().numpy(), ref_gp * k)
    del graph


def test_noalloc_deterministic_is_bitwise(cuda):
    # In the deterministic mode (cpab_set_deterministic) the allocation-free
    # entry point runs the same two passes as cpab_backward: moments and point
    # adjoints equal bit for bit, on two calls in a row, the second smaller.
    # Scaling grad_out by a power of two scales every flushed value and the
    # row's scale exactly, so the moments scale exactly too.
    lib = native()
    for tess, n_theta, nP, batched, seed in (([20, 20], 4, 20000, False, 311),
                                             ([4, 4], 2, 300, True, 312)):
        p, pts, As, g = _case(cuda, tess, n_theta, nP, batched, seed)
        nd, ppc = p.ndim, p.ndim * (p.ndim + 1)
        with lib.deterministic(True):
            ref_m = torch.empty((n_theta, p.nC, ppc), device=cuda)
            ref_gp = torch.empty((n_theta, nd, nP), device=cuda)
            ws = torch.empty(lib.backward_workspace_size(nd, nP, n_theta, p.nC),
                             dtype=torch.uint8, device=cuda)
            lib.backward(nd, pts, batched, n_theta, nP, 50, p.nc, 0, As, g, ref_m, ref_gp, ws)
            m = torch.full((n_theta, p.nC, ppc), 7.0, device=cuda)
            gp = torch.full((n_theta, nd, nP), -3.0, device=cuda)
            lib.backward_noalloc(nd, pts, batched, n_theta, nP, 50, p.nc, 0, As, g, m, gp)
            m4 = torch.empty_like(m)
            lib.backward_noalloc(nd, pts, batched, n_theta, nP, 50, p.nc, 0, As, g * 4.0, m4,
                                 torch.empty_like(gp))
        torch.cuda.synchronize()
        assert torch.equal(m, ref_m) and torch.equal(gp, ref_gp)
        assert torch.equal(m4, m * 4.0)
