"""Kernel-level parity: HIP library (through its C ABI) vs the CPU oracle on the
same seeded inputs.  Bit-exact for the fixed-step integrators, cell sequences,
the 1D closed form, affine map, expm and projection; within tolerance for the
moment sums (float atomics, no fixed order, and the factored reverse sweep),
the point adjoints (factored reverse sweep) and the interpolation backward."""
import numpy as np
import pytest
import torch

from cpab.pytorch._native import native
from cpab.pytorch.transformer import basis_tables
from oracle import oracle as orc

import edge_bound as eb
from helpers import (assert_adjoint_close, assert_grad_close, cpab_for, edge_lattice, meshgrid,
                     recover_growth, scatter_magnitude, seeded_theta, uniform_points)

pytestmark = pytest.mark.gpu


def _dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _As_gpu(T, theta, cuda):
    p = T.params
    tab = basis_tables(p, cuda)
    As = torch.empty((theta.shape[0], p.nC, p.ndim, p.ndim + 1), device=cuda)
    native().affine(p.ndim, _dev(theta, cuda), p.nC, tab["row_ptr"], tab["col_idx"], tab["vals"], As)
    return As


@pytest.mark.parametrize("tess", [[50], [20, 20], [4, 3], [3, 4, 2], [10, 10, 10]])
def test_affine_and_expm_bitexact(cuda, tess):
    T = cpab_for(tess)
    nd = len(tess)
    theta = seeded_theta(T, 4, 0.5, 100 + nd)
    As = _As_gpu(T, theta, cuda)
    ref = orc.affine(theta, T.params.basis).reshape(As.shape)
    np.testing.assert_array_equal(As.cpu().numpy(), ref)
    Tr = torch.empty_like(As)
    native().expm(nd, As, 1.0 / 50, Tr)
    np.testing.assert_array_equal(Tr.cpu().numpy(), orc.expm(nd, ref, 1.0 / 50))
    # The fused launch the forward uses: the same two tables, bit for bit.
    tab = basis_tables(T.params, cuda)
    As2, Tr2 = torch.empty_like(As), torch.empty_like(As)
    native().affine_expm(nd, _dev(theta, cuda), T.params.nC, tab["row_ptr"], tab["col_idx"],
                         tab["vals"], 1.0 / 50, As2, Tr2)
    np.testing.assert_array_equal(As2.cpu().numpy(), ref)
    np.testing.assert_array_equal(Tr2.cpu().numpy(), Tr.cpu().numpy())


def test_expm_squaring_branch_bitexact(cuda):
    # Large |A| exercises the scaling-and-squaring branch (norm > 0.5).
    rng = np.random.default_rng(5)
    for nd in (1, 2, 3):
        A = (rng.standard_normal((257, nd, nd + 1)) * 40).astype(np.float32)
        out = torch.empty(A.shape, device=cuda)
        native().expm(nd, _dev(A, cuda), 0.5, out)
        np.testing.assert_array_equal(out.cpu().numpy(), orc.expm(nd, A, 0.5))


def _forward_case(T, theta, pts, cuda, nstep=50, adaptive=0):
    p = T.params
    nd = p.ndim
    As = _As_gpu(T, theta, cuda)
    Tr = torch.empty_like(As)
    native().expm(nd, As, 1.0 / nstep, Tr)
    pts_d = _dev(pts, cuda)
    batched = pts.ndim == 3
    nP = pts.shape[-1]
    out = torch.empty((theta.shape[0], nd, nP), device=cuda)
    native().forward(nd, pts_d, batched, theta.shape[0], nP, nstep, p.nc, adaptive, Tr, As, out)
    cells = torch.empty((theta.shape[0], nP, nstep), dtype=torch.int32, device=cuda)
    native().trace_cells(nd, pts_d, batched, theta.shape[0], nP, nstep, p.nc, adaptive, Tr, As, cells)
    return As.cpu().numpy(), Tr.cpu().numpy(), out.cpu().numpy(), cells.cpu().numpy()


@pytest.mark.parametrize("adaptive", [0, 1])
@pytest.mark.parametrize("tess,pts_kind", [([20, 20], "uniform"), ([16, 16], "mesh"),
                                           ([30, 30], "mesh"), ([3, 5], "outside")])
def test_forward_2d_bitexact(cuda, tess, pts_kind, adaptive):
    T = cpab_for(tess)
    theta = seeded_theta(T, 3, 0.5, 22)
    if pts_kind == "uniform":
        pts = uniform_points(2, 20000, 21)
    elif pts_kind == "mesh":
        pts = meshgrid([96, 80])
    else:  # points outside the domain exercise the boundary-triangle rules
        pts = (uniform_points(2, 20000, 3) * 1.6 - 0.3).astype(np.float32)
    As, Tr, out, cells = _forward_case(T, theta, pts, cuda, adaptive=adaptive)
    ref, ref_cells = orc.forward_trels(pts, Tr, As, tess, 50, adaptive=bool(adaptive),
                                       return_cells=True)
    np.testing.assert_array_equal(cells, ref_cells)
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("adaptive", [0, 1])
@pytest.mark.parametrize("tess", [[20, 20], [30, 30], [3, 5]])
def test_forward_2d_edge_ties(cuda, tess, adaptive):
    # The lookup skips the out-of-domain rules when every outside lane already
    # has its side's triangle from the inside rule; corners and cell-edge ties
    # on the domain boundary must still come out as the reference's rules say.
    T = cpab_for(tess)
    theta = seeded_theta(T, 2, 0.5, 24)
    pts = edge_lattice(tess, 25)
    As, Tr, out, cells = _forward_case(T, theta, pts, cuda, adaptive=adaptive)
    ref, ref_cells = orc.forward_trels(pts, Tr, As, tess, 50, adaptive=bool(adaptive),
                                       return_cells=True)
    np.testing.assert_array_equal(cells, ref_cells)
    np.testing.assert_array_equal(out, ref)
    g = np.random.default_rng(26).standard_normal((2, 2, pts.shape[1])).astype(np.float32)
    _, mom, gp = _backward_case(T, theta, pts, g, cuda, adaptive=adaptive)
    ref_m, ref_gp = orc.backward(pts, As, g, tess, 50, adaptive=bool(adaptive))
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("tess", [[20, 20], [3, 5], [4, 3, 5]])
def test_forward_nan_inf_points(cuda, tess):
    # NaN and infinite coordinates, alone or beside ordinary ones: the lookup
    # clamps NaN to 0 (fminf(fmaxf(NaN, 0), hi) in the reference; the device's
    # v_med3_f32 returns its smallest operand when one is NaN) and fails every
    # outside test with it, and clamps infinities to the domain.  Visited cells
    # exact, coordinates equal (NaN where the reference's are).
    T = cpab_for(tess)
    theta = seeded_theta(T, 2, 0.5, 48)
    nd = len(tess)
    special = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.3, 0.0, 1.0, -0.2, 1.2], np.float32)
    axes = np.meshgrid(*([special] * nd), indexing="ij")
    pts = np.stack([a.ravel() for a in axes]).astype(np.float32)
    As, Tr, out, cells = _forward_case(T, theta, pts, cuda)
    ref, ref_cells = orc.forward_trels(pts, Tr, As, tess, 50, return_cells=True)
    np.testing.assert_array_equal(cells, ref_cells)
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("adaptive", [0, 1])
@pytest.mark.parametrize("tess", [[4, 3, 5], [10, 10, 10]])
def test_forward_3d_edge_lattice(cuda, tess, adaptive):
    # Points on and beyond faces, edges and corners: the clamping path, the
    # corner rule behind its prefilter, and the visited cells as the
    # reference's rules give them.
    T = cpab_for(tess)
    theta = seeded_theta(T, 2, 0.5, 47)
    pts = edge_lattice(tess, 27)
    As, Tr, out, cells = _forward_case(T, theta, pts, cuda, adaptive=adaptive)
    ref, ref_cells = orc.forward_trels(pts, Tr, As, tess, 50, adaptive=bool(adaptive),
                                       return_cells=True)
    np.testing.assert_array_equal(cells, ref_cells)
    np.testing.assert_array_equal(out, ref)
    g = np.random.default_rng(28).standard_normal((2, 3, pts.shape[1])).astype(np.float32)
    _, mom, gp = _backward_case(T, theta, pts, g, cuda, adaptive=adaptive)
    ref_m, ref_gp = orc.backward(pts, As, g, tess, 50, adaptive=bool(adaptive))
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("adaptive", [0, 1])
@pytest.mark.parametrize("tess,pts_kind", [([4, 4, 4], "mesh"), ([10, 10, 10], "uniform"),
                                           ([2, 3, 2], "outside")])
def test_forward_3d_bitexact(cuda, tess, pts_kind, adaptive):
    T = cpab_for(tess)
    theta = seeded_theta(T, 2, 0.5, 43)
    if pts_kind == "mesh":
        pts = meshgrid([21, 17, 13])
    elif pts_kind == "uniform":
        pts = uniform_points(3, 8000, 41)
    else:
        pts = (uniform_points(3, 8000, 4) * 1.6 - 0.3).astype(np.float32)
    As, Tr, out, cells = _forward_case(T, theta, pts, cuda, adaptive=adaptive)
    ref, ref_cells = orc.forward_trels(pts, Tr, As, tess, 50, adaptive=bool(adaptive),
                                       return_cells=True)
    np.testing.assert_array_equal(cells, ref_cells)
    np.testing.assert_array_equal(out, ref)


def test_forward_batched_points(cuda):
    T = cpab_for([20, 20])
    theta = seeded_theta(T, 3, 0.5, 9)
    pts = np.random.default_rng(8).random((3, 2, 5000)).astype(np.float32)
    As, Tr, out, cells = _forward_case(T, theta, pts, cuda)
    ref = orc.forward_trels(pts, Tr, As, [20, 20], 50)
    np.testing.assert_array_equal(out, ref)


def test_forward_1d_closed_form(cuda):
    T = cpab_for([50])
    theta = seeded_theta(T, 16, 0.5, 11)
    pts = np.linspace(0, 1, 10000, dtype=np.float32)[None]
    As = _As_gpu(T, theta, cuda)
    out = torch.empty((16, 1, 10000), device=cuda)
    native().forward_1d_closed_form(_dev(pts, cuda), False, 16, 10000, 50, As, out)
    ref = orc.forward_closed_1d(pts, As.cpu().numpy(), [50])
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def _backward_case(T, theta, pts, g, cuda, nstep=50, adaptive=0, want_points=True):
    p = T.params
    nd = p.ndim
    As = _As_gpu(T, theta, cuda)
    n_theta, nP = theta.shape[0], pts.shape[-1]
    mom = torch.empty((n_theta, p.nC, nd * (nd + 1)), device=cuda)
    gp = torch.empty((n_theta, nd, nP), device=cuda) if want_points else None
    nbytes = native().backward_workspace_size(nd, nP, n_theta, p.nC)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda) if nbytes else None
    native().backward(nd, _dev(pts, cuda), pts.ndim == 3, n_theta, nP, nstep, p.nc, adaptive, As,
                      _dev(g, cuda), mom, gp, ws)
    return As.cpu().numpy(), mom.cpu().numpy(), None if gp is None else gp.cpu().numpy()


@pytest.mark.parametrize("adaptive", [0, 1])
@pytest.mark.parametrize("tess,kind,n", [([50], "line", 10000), ([20, 20], "uniform", 20000),
                                         ([30, 30], "mesh", 0), ([10, 10, 10], "uniform", 6000),
                                         ([4, 4, 4], "mesh", 0)])
def test_backward_parity(cuda, tess, kind, n, adaptive):
    T = cpab_for(tess)
    nd = len(tess)
    theta = seeded_theta(T, 3, 0.5, 60 + nd)
    if kind == "line":
        pts = np.linspace(0, 1, n, dtype=np.float32)[None]
    elif kind == "uniform":
        pts = uniform_points(nd, n, 61)
    else:
        pts = meshgrid([64, 48] if nd == 2 else [17, 13, 11])
    g = np.random.default_rng(62).standard_normal((3, nd, pts.shape[-1])).astype(np.float32)
    As, mom, gp = _backward_case(T, theta, pts, g, cuda, adaptive=adaptive)
    ref_m, ref_gp = orc.backward(pts, As, g, tess, 50, adaptive=bool(adaptive))
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("tess,scale", [([20, 20], 0.5), ([6, 5], 1.0), ([16, 16], 2.0)])
def test_backward_edge_bound_start_points(cuda, tess, scale):
    # 2D register backward: a wave whose lanes all start at least the row's
    # bound delta_T (restated in tests/edge_bound.py) from every edge replays
    # without the lookup's edge test.  Points at the largest row bound, one
    # float closer, and 1.01x further, along every edge, in runs of whole waves,
    # beside uniform points and the edge lattice: moments and point adjoints
    # against the oracle (a wrong cell at any step would move the adjoint far
    # outside its tolerance).  At scale 2 some rows have no bound.
    T = cpab_for(tess)
    p = T.params
    nx, ny = p.nc
    theta = seeded_theta(T, 3, scale, 140)
    A = orc.affine(theta, p.basis).reshape(3, p.nC, 2, 3)
    deltas = np.array([eb.midpoint_delta(A[b], 50, nx, ny) for b in range(3)])
    if scale <= 0.5:
        assert np.isfinite(deltas).all(), deltas
    finite = deltas[np.isfinite(deltas)]
    rng = np.random.default_rng(141)
    parts = [uniform_points(2, 8192, 142), edge_lattice(tess, 143)]
    for d in (finite.max(), np.nextafter(np.float32(finite.max()), np.float32(0)),
              np.float32(1.01) * finite.max()) if finite.size else ():
        d = np.float32(d)
        for side in range(4):
            u = rng.random(256).astype(np.float32)
            fixed = np.full(256, d if side % 2 == 0 else np.float32(1) - d, np.float32)
            parts.append(np.stack((fixed, u) if side < 2 else (u, fixed)))
    pts = np.concatenate(parts, axis=1).astype(np.float32)
    g = rng.standard_normal((3, 2, pts.shape[1])).astype(np.float32)
    As, mom, gp = _backward_case(T, theta, pts, g, cuda)
    np.testing.assert_array_equal(As, A)
    ref_m, ref_gp = orc.backward(pts, As, g, tess, 50)
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("tess,kind,scale,recovered", [
    # growth bound (max ||M_c||_2)^50 at most 16: positions recovered through
    # the inverse one-step maps, up to the bound
    ([20, 20], "uniform", 1.0, True), ([50], "line", 1.0, True), ([4, 4, 4], "mesh", 1.5, True),
    ([10, 10, 10], "uniform", 1.7, True),
    # beyond it: every segment replayed from a checkpoint (exact positions)
    ([20, 20], "uniform", 2.0, False), ([30, 30], "mesh", 2.0, False), ([50], "line", 3.0, False),
    ([50], "line", 6.0, False), ([50], "line", 10.0, False), ([20, 20], "uniform", 4.0, False),
    ([20, 20], "uniform", 8.0, False), ([16, 16], "mesh", 6.0, False),
    ([4, 4, 4], "mesh", 8.0, False), ([10, 10, 10], "uniform", 6.0, False)])
def test_backward_parity_strong_field(cuda, tess, kind, scale, recovered):
    # Large theta: strong, fast-changing fields, where the factored adjoint sees
    # the largest h*|A| and where recovering positions backwards through the
    # inverse maps would amplify their rounding by up to (max ||M_c||_2)^T
    # (1e4 .. 1e7 at the strongest cases here: errors of 1e-3 .. 0.4 in the
    # positions).  The library recovers positions only below a bound of 16 and
    # otherwise replays each segment from a checkpoint; `recovered` records
    # which side of the bound each case sits on, so both paths are covered.
    T = cpab_for(tess)
    nd = len(tess)
    theta = seeded_theta(T, 2, scale, 110 + nd)
    if kind == "line":
        pts = np.linspace(0, 1, 5000, dtype=np.float32)[None]
    elif kind == "uniform":
        pts = uniform_points(nd, 20000, 111)
    else:
        pts = meshgrid([64, 48] if nd == 2 else [17, 13, 11])
    g = np.random.default_rng(112).standard_normal((2, nd, pts.shape[-1])).astype(np.float32)
    As, mom, gp = _backward_case(T, theta, pts, g, cuda)
    growth = recover_growth(As)
    assert ((growth <= 16.0).all() if recovered else (growth > 16.0).all()), growth
    ref_m, ref_gp = orc.backward(pts, As, g, tess, 50)
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("tess,kind,nstep", [([50], "line", 20), ([20, 20], "uniform", 37),
                                             ([30, 30], "mesh", 100), ([4, 4, 4], "uniform", 20),
                                             ([10, 10, 10], "mesh", 37)])
def test_backward_segmented_steps(cuda, tess, kind, nstep):
    # nstepsolver != 50 runs the segmented replay (a checkpoint every 8 steps,
    # replayed per segment; 37 and 20 leave a partial last segment; 100 is the
    # step cap).
    T = cpab_for(tess)
    nd = len(tess)
    theta = seeded_theta(T, 2, 0.5, 90 + nd)
    if kind == "line":
        pts = np.linspace(0, 1, 4000, dtype=np.float32)[None]
    elif kind == "uniform":
        pts = uniform_points(nd, 6000, 91)
    else:
        pts = meshgrid([48, 40] if nd == 2 else [23, 19, 17])
    g = np.random.default_rng(92).standard_normal((2, nd, pts.shape[-1])).astype(np.float32)
    As, mom, gp = _backward_case(T, theta, pts, g, cuda, nstep=nstep)
    ref_m, ref_gp = orc.backward(pts, As, g, tess, nstep)
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("kind,n", [("mesh", 0), ("uniform", 120000)])
def test_backward_3d_moment_paths(cuda, kind, n):
    # [10,10,10]: the 5000 x 12 moment table does not fit in LDS, so sums go to
    # the hashed LDS cell cache: meshgrid points keep the cells of a workgroup
    # few; 120k uniform points under one theta touch more distinct cells per
    # workgroup than the cache has slots, so flushes also take the HBM
    # fallback.
    T = cpab_for([10, 10, 10])
    theta = seeded_theta(T, 1, 0.5, 71)
    pts = meshgrid([40, 36, 30]) if kind == "mesh" else uniform_points(3, n, 72)
    g = np.random.default_rng(73).standard_normal((1, 3, pts.shape[-1])).astype(np.float32)
    As, mom, gp = _backward_case(T, theta, pts, g, cuda)
    ref_m, ref_gp = orc.backward(pts, As, g, [10, 10, 10], 50)
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


def _random_field_case(nc, n_theta, nP, scale, seed, mesh=None):
    """Per-cell fields drawn independently (no basis: the kernels take any
    table), for tessellations too large to build a basis for in a test."""
    nd = len(nc)
    nC = {1: nc[0], 2: 4 * nc[0] * nc[1], 3: 5 * int(np.prod(nc))}[nd]
    rng = np.random.default_rng(seed)
    As = (rng.standard_normal((n_theta, nC, nd, nd + 1)) * scale).astype(np.float32)
    pts = meshgrid(mesh) if mesh else rng.random((nd, nP)).astype(np.float32)
    g = rng.standard_normal((n_theta, nd, pts.shape[-1])).astype(np.float32)
    return As, pts, g


@pytest.mark.parametrize("nc,mesh,nstep", [
    # 2D table beyond LDS (9216 cells x 6 floats = 221 KiB): the cell cache,
    # segmented variant, for uniform points (cache misses go to HBM) and a mesh
    ([48, 48], None, 50), ([48, 48], [80, 72], 50), ([48, 48], None, 37),
    # 3D with more than 65535 cells: no register variant (16-bit cell ids), so
    # the segmented variant with the cell cache
    ([24, 24, 24], None, 50), ([24, 24, 24], [30, 28, 26], 50)])
def test_backward_large_tessellations(cuda, nc, mesh, nstep):
    nd = len(nc)
    As_np, pts, g = _random_field_case(nc, 2, 20000, 0.4, 170 + nd, mesh)
    nC = As_np.shape[1]
    As = _dev(As_np, cuda)
    Tr = torch.empty_like(As)
    native().expm(nd, As, 1.0 / nstep, Tr)
    nP = pts.shape[-1]
    out = torch.empty((2, nd, nP), device=cuda)
    native().forward(nd, _dev(pts, cuda), False, 2, nP, nstep, nc, 0, Tr, As, out)
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  orc.forward_trels(pts, Tr.cpu().numpy(), As_np, nc, nstep))
    mom = torch.empty((2, nC, nd * (nd + 1)), device=cuda)
    gp = torch.empty((2, nd, nP), device=cuda)
    ws = torch.empty(native().backward_workspace_size(nd, nP, 2, nC), dtype=torch.uint8, device=cuda)
    native().backward(nd, _dev(pts, cuda), False, 2, nP, nstep, nc, 0, As, _dev(g, cuda), mom, gp, ws)
    ref_m, ref_gp = orc.backward(pts, As_np, g, nc, nstep)
    assert_adjoint_close(gp.cpu().numpy(), ref_gp)
    assert_grad_close(mom.cpu().numpy(), ref_m, rtol=2e-5)


@pytest.mark.parametrize("chain", [False, True])
def test_backward_mixed_dense_sparse(cuda, chain):
    # One launch where some workgroups touch most cells (uniform points: they
    # store partial tables) and others touch few (a small cluster: they add
    # their sums to HBM with atomics), into the same moments rows.
    T = cpab_for([20, 20])
    p = T.params
    rng = np.random.default_rng(77)
    spread = rng.random((2, 60000)).astype(np.float32)
    cluster = (0.4 + 0.05 * rng.random((2, 60000))).astype(np.float32)
    pts = np.concatenate([spread, cluster], axis=1)
    nP = pts.shape[1]
    if not chain:
        theta = seeded_theta(T, 2, 0.5, 78)
        g = rng.standard_normal((2, 2, nP)).astype(np.float32)
        As, mom, gp = _backward_case(T, theta, pts, g, cuda)
        ref_m, ref_gp = orc.backward(pts, As, g, [20, 20], 50)
        assert_adjoint_close(gp, ref_gp)
        assert_grad_close(mom, ref_m, rtol=2e-5)
        return
    K = 2
    theta = seeded_theta(T, K, 0.3, 79)
    As = _As_gpu(T, theta, cuda)
    Tr = torch.empty_like(As)
    native().expm(2, As, 1.0 / 50, Tr)
    out = torch.empty((1, 2, nP), device=cuda)
    sp = torch.empty((K - 1, 1, 2, nP), device=cuda)
    native().chain_forward(2, _dev(pts, cuda), False, 1, K, nP, 50, p.nc, 0, Tr, As, out, sp)
    g = rng.standard_normal((1, 2, nP)).astype(np.float32)
    mom = torch.empty((K, p.nC, 6), device=cuda)
    gp = torch.empty((1, 2, nP), device=cuda)
    ws = torch.empty(native().chain_backward_workspace_size(2, nP, 1, K, p.nC), dtype=torch.uint8,
                     device=cuda)
    native().chain_backward(2, _dev(pts, cuda), False, 1, K, nP, 50, p.nc, 0, sp, As, _dev(g, cuda),
                            mom, gp, ws)
    A = As.cpu().numpy().reshape(K, 1, p.nC, 2, 3)
    x1 = sp[0].cpu().numpy()
    m1, lam = orc.backward(x1, A[1], g, [20, 20], 50)
    m0, lam = orc.backward(pts, A[0], lam, [20, 20], 50)
    M = mom.cpu().numpy()
    assert_grad_close(M[1], m1[0], rtol=2e-5)
    assert_grad_close(M[0], m0[0], rtol=2e-5)
    assert_adjoint_close(gp.cpu().numpy(), lam)


@pytest.mark.parametrize("tess,n_theta", [([20, 20], 1), ([50], 2)])
def test_backward_dense_parts_many_words(cuda, tess, n_theta):
    # One or two theta rows over 200,000 uniform points: about 196 (98) point
    # ranges per row, every workgroup dense, so each row's dense-part mask
    # spans several 64-bit words and finish_moments_kernel adds that many
    # partial tables per cell.
    T = cpab_for(tess)
    nd = len(tess)
    theta = seeded_theta(T, n_theta, 0.5, 66)
    pts = uniform_points(nd, 200000, 67)
    g = np.random.default_rng(68).standard_normal((n_theta, nd, pts.shape[-1])).astype(np.float32)
    As, mom, gp = _backward_case(T, theta, pts, g, cuda)
    ref_m, ref_gp = orc.backward(pts, As, g, tess, 50)
    assert_adjoint_close(gp, ref_gp)
    assert_grad_close(mom, ref_m, rtol=2e-5)


def test_backward_no_points_grad(cuda):
    T = cpab_for([20, 20])
    theta = seeded_theta(T, 2, 0.5, 3)
    pts = uniform_points(2, 3000, 4)
    g = np.random.default_rng(5).standard_normal((2, 2, 3000)).astype(np.float32)
    As, mom, _ = _backward_case(T, theta, pts, g, cuda, want_points=False)
    ref_m, _ = orc.backward(pts, As, g, [20, 20], 50)
    assert_grad_close(mom, ref_m, rtol=2e-5)


@pytest.mark.parametrize("tess", [[50], [20, 20], [10, 10, 10]])
def test_project_bitexact(cuda, tess):
    T = cpab_for(tess)
    p = T.params
    tab = basis_tables(p, cuda)
    M = np.random.default_rng(1).standard_normal((5, p.D)).astype(np.float32)
    out = torch.empty((5, p.d), device=cuda)
    native().project(_dev(M, cuda), p.D, p.d, tab["col_ptr"], tab["row_idx"], tab["vals_t"], out)
    np.testing.assert_array_equal(out.cpu().numpy(), orc.project(M, p.basis))


@pytest.mark.parametrize("nd,ins,outs", [(2, (40, 56), (48, 36)), (3, (12, 10, 14), (9, 11, 13)),
                                         (1, (77,), (50,)), (2, (512, 512), (130, 70)),
                                         (2, (64, 80), (96, 130)), (3, (12, 10, 14), (32, 3, 66)),
                                         # last data axis of size 1 or 2 (the whole-tile
                                         # gathers read corner pairs along it when >= 2)
                                         (2, (40, 1), (64, 64)), (3, (12, 10, 1), (32, 4, 32)),
                                         (2, (3, 2), (64, 40)), (3, (5, 3, 2), (32, 2, 32))])
def test_interp_parity(cuda, nd, ins, outs):
    rng = np.random.default_rng(30 + nd)
    B, C = 2, 3
    data = rng.random((B, C, *ins)).astype(np.float32)
    nP = int(np.prod(outs))
    grid = (rng.random((B, nd, nP)) * 1.3 - 0.15).astype(np.float32)  # incl. clamped border
    gout = rng.standard_normal((B, C, *outs)).astype(np.float32)
    out = torch.empty((B, C, *outs), device=cuda)
    native().interp_forward(nd, _dev(data, cuda), _dev(grid, cuda), outs, out)
    np.testing.assert_array_equal(out.cpu().numpy(), orc.interp_forward(nd, data, grid, outs))
    gg = torch.empty((B, nd, nP), device=cuda)
    gd = torch.empty_like(torch.from_numpy(data)).to(cuda)
    native().interp_backward(nd, _dev(data, cuda), _dev(grid, cuda), outs, _dev(gout, cuda), gg, gd)
    # Same fp32 weights and per-point sums as the oracle: grad_grid is bit-exact.
    rg, rd = orc.interp_backward(nd, data, grid, outs, gout)
    np.testing.assert_array_equal(gg.cpu().numpy(), rg)
    # grad_data sums many contributions per pixel with float atomics (clamped
    # border points pile up, several hundred per pixel here) in an order that
    # differs from the oracle's sequential fp32 sum; both round each partial
    # sum, so the difference is bounded by ~(2 count 2^-24) of the pixel's
    # summed contribution magnitudes.
    mag = scatter_magnitude(data.shape, grid, outs, gout)
    err = np.abs(gd.cpu().numpy().astype(np.float64) - rd)
    assert (err <= 1e-4 * mag + 1e-12).all(), float((err / (mag + 1e-30)).max())


@pytest.mark.parametrize("nd,tess,ins,outs", [(2, [6, 5], (150, 210), (96, 160)),
                                              (3, [3, 3, 2], (40, 36, 44), (64, 6, 64))])
def test_interp_smooth_warp(cuda, nd, tess, ins, outs):
    # Resampling at a CPAB-warped meshgrid, as transform_data does: the tiles
    # of a smooth warp read compact data regions (in 2D, full tiles stage that
    # region in LDS; regions that are too large take the direct gathers).  The
    # grid is scaled past [0, 1] at one end so border tiles clamp.
    T = cpab_for(tess)
    B, C = 2, 3
    rng = np.random.default_rng(60 + nd)
    theta = seeded_theta(T, B, 0.8, 61 + nd)
    with torch.no_grad():
        mesh = T.uniform_meshgrid(list(outs))
        grid_t = T.transform_grid(mesh, torch.tensor(theta, device=cuda)) * 1.08 - 0.02
    grid = grid_t.cpu().numpy().astype(np.float32)
    data = rng.random((B, C, *ins)).astype(np.float32)
    out = torch.empty((B, C, *outs), device=cuda)
    native().interp_forward(nd, _dev(data, cuda), _dev(grid, cuda), outs, out)
    np.testing.assert_array_equal(out.cpu().numpy(), orc.interp_forward(nd, data, grid, outs))
    gout = rng.standard_normal((B, C, *outs)).astype(np.float32)
    nP = int(np.prod(outs))
    gg = torch.empty((B, nd, nP), device=cuda)
    native().interp_backward(nd, _dev(data, cuda), _dev(grid, cuda), outs, _dev(gout, cuda), gg, None)
    rg, rd = orc.interp_backward(nd, data, grid, outs, gout)
    np.testing.assert_array_equal(gg.cpu().numpy(), rg)
    gd = torch.empty((B, C, *ins), device=cuda)
    native().interp_backward(nd, _dev(data, cuda), _dev(grid, cuda), outs, _dev(gout, cuda), gg, gd)
    np.testing.assert_array_equal(gg.cpu().numpy(), rg)
    mag = scatter_magnitude(data.shape, grid, outs, gout)
    err = np.abs(gd.cpu().numpy().astype(np.float64) - rd)
    assert (err <= 1e-4 * mag + 1e-12).all(), float((err / (mag + 1e-30)).max())


def test_interp_unaligned_grid(cuda):
    # A grid view that starts 4 bytes into its buffer cannot take the 16-byte
    # vector path; results must not change.
    rng = np.random.default_rng(7)
    outs = (64, 64)
    nP = 64 * 64
    data = rng.random((1, 2, 33, 47)).astype(np.float32)
    grid = (rng.random((1, 2, nP)) * 1.2 - 0.1).astype(np.float32)
    buf = torch.empty(1 + grid.size, device=cuda)
    view = buf[1:].view(1, 2, nP)
    view.copy_(torch.from_numpy(grid))
    out = torch.empty((1, 2, *outs), device=cuda)
    native().interp_forward(2, _dev(data, cuda), view, outs, out)
    np.testing.assert_array_equal(out.cpu().numpy(), orc.interp_forward(2, data, grid, outs))
    gout = rng.standard_normal((1, 2, *outs)).astype(np.float32)
    gbuf = torch.empty(1 + grid.size, device=cuda)
    gg = gbuf[1:].view(1, 2, nP)
    native().interp_backward(2, _dev(data, cuda), view, outs, _dev(gout, cuda), gg, None)
    rg, _ = orc.interp_backward(2, data, grid, outs, gout)
    np.testing.assert_array_equal(gg.cpu().numpy(), rg)


@pytest.mark.parametrize("tess,kind,adaptive,scale", [([50], "line", 0, 0.3), ([16, 16], "mesh", 0, 0.3),
                                                      ([16, 16], "batched", 1, 0.3),
                                                      ([4, 4, 4], "uniform", 0, 0.3),
                                                      ([10, 10, 10], "mesh", 0, 0.3),
                                                      # strong stages: checkpoint replay
                                                      ([16, 16], "mesh", 0, 5.0),
                                                      ([50], "line", 0, 6.0)])
def test_chain_matches_stagewise(cuda, tess, kind, adaptive, scale):
    # cpab_chain_forward / cpab_chain_backward against the stage-by-stage
    # composition the reference's transform_grid_chain performs
    # (cpab/cpab.py:270-278): stage outputs and stage inputs bit-exact; the
    # adjoint handed from stage to stage (grad_points) and the moments of every
    # stage within tolerance.
    T = cpab_for(tess)
    p = T.params
    nd = len(tess)
    K, nb = 3, 2
    theta = (np.random.default_rng(81).standard_normal((K * nb, p.d)) * scale).astype(np.float32)
    if kind == "line":
        pts = np.linspace(0, 1, 3000, dtype=np.float32)[None]
    elif kind == "mesh":
        pts = meshgrid([40, 32] if nd == 2 else [17, 13, 11])
    elif kind == "batched":
        pts = np.random.default_rng(82).random((nb, nd, 4000)).astype(np.float32)
    else:
        pts = uniform_points(nd, 5000, 83)
    batched = pts.ndim == 3
    nP = pts.shape[-1]
    As = _As_gpu(T, theta, cuda)
    Tr = torch.empty_like(As)
    native().expm(nd, As, 1.0 / 50, Tr)
    out = torch.empty((nb, nd, nP), device=cuda)
    sp = torch.empty((K - 1, nb, nd, nP), device=cuda)
    native().chain_forward(nd, _dev(pts, cuda), batched, nb, K, nP, 50, p.nc, adaptive, Tr, As,
                           out, sp)
    A = As.cpu().numpy().reshape(K, nb, p.nC, nd, nd + 1)
    R = Tr.cpu().numpy().reshape(K, nb, p.nC, nd, nd + 1)
    if scale > 1.0:
        assert (recover_growth(A.reshape(K * nb, p.nC, nd, nd + 1)) > 16.0).all()
    xs = [pts]
    for s in range(K):
        if nd == 1:
            xs.append(orc.forward_closed_1d(xs[-1], A[s], p.nc))
        else:
            xs.append(orc.forward_trels(xs[-1], R[s], A[s], p.nc, 50, adaptive=bool(adaptive)))
    np.testing.assert_array_equal(out.cpu().numpy(), xs[-1])
    for s in range(1, K):
        np.testing.assert_array_equal(sp[s - 1].cpu().numpy(), xs[s])

    g = np.random.default_rng(84).standard_normal((nb, nd, nP)).astype(np.float32)
    mom = torch.empty((K * nb, p.nC, nd * (nd + 1)), device=cuda)
    gp = torch.empty((nb, nd, nP), device=cuda)
    nbytes = native().chain_backward_workspace_size(nd, nP, nb, K, p.nC)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda) if nbytes else None
    native().chain_backward(nd, _dev(pts, cuda), batched, nb, K, nP, 50, p.nc, adaptive, sp, As,
                            _dev(g, cuda), mom, gp, ws)
    M = mom.cpu().numpy().reshape(K, nb, p.nC, -1)
    lam = g
    for s in reversed(range(K)):
        ref_m, lam = orc.backward(xs[s], A[s], lam, p.nc, 50, adaptive=bool(adaptive))
        assert_grad_close(M[s], ref_m, rtol=2e-5)
    assert_adjoint_close(gp.cpu().numpy(), lam)


def _image_order(x, outs):
    """[B, nd, prod(outs)] in meshgrid order (coordinate 0 fastest) -> image order
    (last axis fastest), the layout of cpab_transform_data_forward's final points."""
    B, nd = x.shape[:2]
    sp = x.reshape(B, nd, *outs[::-1])
    return np.ascontiguousarray(sp.transpose(0, 1, *range(nd + 1, 1, -1))).reshape(B, nd, -1)


@pytest.mark.parametrize("tess,ins,outs,adaptive,scale", [([10], (50,), (70,), 0, 0.5),
                                                          ([6, 5], (40, 48), (36, 44), 0, 0.5),
                                                          ([6, 5], (40, 48), (36, 44), 1, 0.5),
                                                          ([3, 3, 3], (10, 12, 9), (11, 9, 13), 0, 0.5),
                                                          # last axis % 16 == 0 and the one before
                                                          # % 4 == 0: the tiled walk
                                                          ([6, 5], (40, 48), (36, 48), 0, 0.5),
                                                          ([6, 5], (40, 48), (20, 32), 1, 0.5),
                                                          ([3, 3, 3], (10, 12, 9), (6, 8, 32), 0, 0.5),
                                                          # strong fields: checkpoint replay
                                                          ([6, 5], (40, 48), (36, 48), 0, 5.0),
                                                          ([3, 3, 3], (10, 12, 9), (6, 8, 32), 0, 8.0),
                                                          ([10], (50,), (70,), 0, 6.0)])
def test_transform_data_fused_parity(cuda, tess, ins, outs, adaptive, scale):
    # cpab_transform_data_forward / _backward against the unfused composition
    # the reference runs (transform_grid of the meshgrid, interpolate, and the
    # autograd backward through both): image and final points bit-exact,
    # moments and grad_data within tolerance.
    T = cpab_for(tess)
    p = T.params
    nd = len(tess)
    B, C = 2, 2
    theta = seeded_theta(T, B, scale, 91)
    rng = np.random.default_rng(92)
    data = rng.random((B, C, *ins)).astype(np.float32)
    grid = T.uniform_meshgrid(list(outs))
    grid_np = grid.cpu().numpy()
    # the fused entry points take the grid's per-axis coordinates; their
    # Cartesian product (coordinate 0 fastest) is the meshgrid
    axes = T._uniform_axes(list(outs))
    ax_np = axes.cpu().numpy()
    offs = np.cumsum([0] + list(outs))
    for k in range(nd):
        ik = (np.arange(int(np.prod(outs))) // int(np.prod(outs[:k]))) % outs[k]
        np.testing.assert_array_equal(ax_np[offs[k] + ik], grid_np[k])
    As = _As_gpu(T, theta, cuda)
    if scale > 1.0:
        assert (recover_growth(As.cpu().numpy()) > 16.0).all()
    Tr = torch.empty_like(As)
    native().expm(nd, As, 1.0 / 50, Tr)
    out = torch.empty((B, C, *outs), device=cuda)
    nP = int(np.prod(outs))
    fin = torch.empty((B, nd, nP), device=cuda)
    native().transform_data_forward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, adaptive,
                                    Tr, As, out, fin)
    A = As.cpu().numpy()
    if nd == 1:
        xT = orc.forward_closed_1d(grid_np, A, p.nc)
    else:
        xT = orc.forward_trels(grid_np, Tr.cpu().numpy(), A, p.nc, 50, adaptive=bool(adaptive))
    np.testing.assert_array_equal(fin.cpu().numpy(), _image_order(xT, outs))
    np.testing.assert_array_equal(out.cpu().numpy(), orc.interp_forward(nd, data, xT, outs))

    gout = rng.standard_normal((B, C, *outs)).astype(np.float32)
    mom = torch.empty((B, p.nC, nd * (nd + 1)), device=cuda)
    gd = torch.empty((B, C, *ins), device=cuda)
    nbytes = native().transform_data_backward_workspace_size(nd, B, list(outs), p.nC)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda) if nbytes else None
    native().transform_data_backward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, adaptive,
                                     fin, As, _dev(gout, cuda), mom, gd, ws)
    rg, rd = orc.interp_backward(nd, data, xT, outs, gout)
    ref_m, _ = orc.backward(grid_np, A, rg, p.nc, 50, adaptive=bool(adaptive))
    assert_grad_close(mom.cpu().numpy(), ref_m, rtol=2e-5)
    mag = scatter_magnitude(data.shape, xT, outs, gout)
    err = np.abs(gd.cpu().numpy().astype(np.float64) - rd)
    assert (err <= 1e-4 * mag + 1e-12).all(), float((err / (mag + 1e-30)).max())


@pytest.mark.parametrize("tess,ins,outs,scale", [([10], (50,), (70,), 0.5),
                                                 ([6, 5], (40, 48), (36, 48), 0.5),
                                                 ([6, 5], (37, 23), (29, 31), 0.5),
                                                 ([3, 3, 3], (10, 12, 9), (6, 8, 32), 0.5),
                                                 ([6, 5], (40, 48), (36, 48), 5.0)])
def test_transform_data_seed_grad(cuda, tess, ins, outs, scale):
    # One channel: the forward also writes the sample's spatial gradient at each
    # final point, and the backward seeds from it (no final points, no data
    # reads).  The image is bit-exact; the stored gradient times (size - 1) is
    # the resampling backward's grad_grid at unit image gradient, bit for bit
    # (blend_grad with g = 1 multiplies by 1); the moments match the oracle and
    # the final-point path within the backward's tolerance.
    T = cpab_for(tess)
    p = T.params
    nd = len(tess)
    B = 2
    theta = seeded_theta(T, B, scale, 95)
    rng = np.random.default_rng(96)
    data = rng.random((B, 1, *ins)).astype(np.float32)
    grid_np = T.uniform_meshgrid(list(outs)).cpu().numpy()
    axes = T._uniform_axes(list(outs))
    As = _As_gpu(T, theta, cuda)
    Tr = torch.empty_like(As)
    native().expm(nd, As, 1.0 / 50, Tr)
    nP = int(np.prod(outs))
    out = torch.empty((B, 1, *outs), device=cuda)
    fin = torch.empty((B, nd, nP), device=cuda)
    sg = torch.empty((B, nd, nP), device=cuda)
    native().transform_data_forward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, 0, Tr, As,
                                    out, fin, seed_grad=sg)
    A = As.cpu().numpy()
    if nd == 1:
        xT = orc.forward_closed_1d(grid_np, A, p.nc)
    else:
        xT = orc.forward_trels(grid_np, Tr.cpu().numpy(), A, p.nc, 50)
    np.testing.assert_array_equal(fin.cpu().numpy(), _image_order(xT, outs))
    np.testing.assert_array_equal(out.cpu().numpy(), orc.interp_forward(nd, data, xT, outs))
    unit, _ = orc.interp_backward(nd, data, xT, outs, np.ones((B, 1, *outs), np.float32))
    scale_k = np.array([s_ - 1 for s_ in ins], np.float32).reshape(1, nd, 1)
    np.testing.assert_array_equal(sg.cpu().numpy() * scale_k, _image_order(unit, outs))

    gout = rng.standard_normal((B, 1, *outs)).astype(np.float32)
    nbytes = native().transform_data_backward_workspace_size(nd, B, list(outs), p.nC)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda) if nbytes else None
    mom = torch.empty((B, p.nC, nd * (nd + 1)), device=cuda)
    native().transform_data_backward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, 0, None,
                                     As, _dev(gout, cuda), mom, None, ws, seed_grad=sg)
    rg, _ = orc.interp_backward(nd, data, xT, outs, gout)
    ref_m, _ = orc.backward(grid_np, A, rg, p.nc, 50)
    assert_grad_close(mom.cpu().numpy(), ref_m, rtol=2e-5)
    mom_fin = torch.empty_like(mom)
    native().transform_data_backward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, 0, fin,
                                     As, _dev(gout, cuda), mom_fin, None, ws)
    assert_grad_close(mom.cpu().numpy(), mom_fin.cpu().numpy(), rtol=2e-5)


@pytest.mark.parametrize("case", ["dense", "sparse", "cache3d", "chain", "image"])
def test_fused_projection_matches_project(cuda, case):
    # The backward entry points with a basis table finish each row's moments
    # and then project them onto the basis (two launches after the sweep); the
    # projection must equal cpab_project of the same moments bit for bit (same
    # summation order), and the moments the oracle's within the backward's
    # tolerance.
    tess = {"dense": [20, 20], "sparse": [16, 16], "cache3d": [10, 10, 10], "chain": [16, 16],
            "image": [6, 5]}[case]
    T = cpab_for(tess)
    p = T.params
    nd = len(tess)
    tab = basis_tables(p, cuda)
    ppc = nd * (nd + 1)

    def project(mom):
        gt = torch.empty((mom.shape[0], tab["d"]), device=cuda)
        native().project(mom.view(mom.shape[0], -1), tab["D"], tab["d"], tab["col_ptr"],
                         tab["row_idx"], tab["vals_t"], gt)
        return gt

    if case in ("dense", "sparse", "cache3d"):
        n_theta = 3
        theta = seeded_theta(T, n_theta, 0.5, 260)
        pts = (uniform_points(nd, 30000, 261) if case != "sparse" else meshgrid([96, 80]))
        g = np.random.default_rng(262).standard_normal((n_theta, nd, pts.shape[-1])).astype(np.float32)
        As = _As_gpu(T, theta, cuda)
        nP = pts.shape[-1]
        mom = torch.empty((n_theta, p.nC, ppc), device=cuda)
        gth = torch.empty((n_theta, tab["d"]), device=cuda)
        gp = torch.empty((n_theta, nd, nP), device=cuda)
        ws = torch.empty(native().backward_workspace_size(nd, nP, n_theta, p.nC), dtype=torch.uint8,
                         device=cuda)
        native().backward_project(nd, _dev(pts, cuda), False, n_theta, nP, 50, p.nc, 0, As,
                                  _dev(g, cuda), tab, mom, gth, gp, ws)
        ref_m, ref_gp = orc.backward(pts, As.cpu().numpy(), g, p.nc, 50)
        assert_adjoint_close(gp.cpu().numpy(), ref_gp)
    elif case == "chain":
        K, nb = 4, 2
        theta = (np.random.default_rng(263).standard_normal((K * nb, p.d)) * 0.3).astype(np.float32)
        pts = meshgrid([64, 48])
        nP = pts.shape[-1]
        As = _As_gpu(T, theta, cuda)
        Tr = torch.empty_like(As)
        native().expm(nd, As, 1.0 / 50, Tr)
        out = torch.empty((nb, nd, nP), device=cuda)
        sp = torch.empty((K - 1, nb, nd, nP), device=cuda)
        native().chain_forward(nd, _dev(pts, cuda), False, nb, K, nP, 50, p.nc, 0, Tr, As, out, sp)
        g = np.random.default_rng(264).standard_normal((nb, nd, nP)).astype(np.float32)
        mom = torch.empty((K * nb, p.nC, ppc), device=cuda)
        gth = torch.empty((K * nb, tab["d"]), device=cuda)
        ws = torch.empty(native().chain_backward_workspace_size(nd, nP, nb, K, p.nC),
                         dtype=torch.uint8, device=cuda)
        native().chain_backward(nd, _dev(pts, cuda), False, nb, K, nP, 50, p.nc, 0, sp, As,
                                _dev(g, cuda), mom, None, ws, tab=tab, grad_theta=gth)
        A = As.cpu().numpy().reshape(K, nb, p.nC, nd, nd + 1)
        xs = [pts] + [sp[s].cpu().numpy() for s in range(K - 1)]
        lam, refs = g, [None] * K
        for s in reversed(range(K)):
            refs[s], lam = orc.backward(xs[s], A[s], lam, p.nc, 50)
        ref_m = np.concatenate(refs)
    else:
        B, C, ins, outs = 2, 2, (40, 48), (36, 48)
        theta = seeded_theta(T, B, 0.5, 265)
        rng = np.random.default_rng(266)
        data = rng.random((B, C, *ins)).astype(np.float32)
        axes = T._uniform_axes(list(outs))
        As = _As_gpu(T, theta, cuda)
        Tr = torch.empty_like(As)
        native().expm(nd, As, 1.0 / 50, Tr)
        nP = int(np.prod(outs))
        out = torch.empty((B, C, *outs), device=cuda)
        fin = torch.empty((B, nd, nP), device=cuda)
        native().transform_data_forward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, 0, Tr, As,
                                        out, fin)
        gout = rng.standard_normal((B, C, *outs)).astype(np.float32)
        mom = torch.empty((B, p.nC, ppc), device=cuda)
        gth = torch.empty((B, tab["d"]), device=cuda)
        ws = torch.empty(native().transform_data_backward_workspace_size(nd, B, list(outs), p.nC),
                         dtype=torch.uint8, device=cuda)
        native().transform_data_backward(nd, _dev(data, cuda), axes, list(outs), 50, p.nc, 0, fin,
                                         As, _dev(gout, cuda), mom, None, ws, tab=tab,
                                         grad_theta=gth)
        grid = T.uniform_meshgrid(list(outs)).cpu().numpy()
        xT = orc.forward_trels(grid, Tr.cpu().numpy(), As.cpu().numpy(), p.nc, 50)
        rg, _ = orc.interp_backward(nd, data, xT, outs, gout, want_data=False)
        ref_m, _ = orc.backward(grid, As.cpu().numpy(), rg, p.nc, 50)
    assert_grad_close(mom.cpu().numpy(), ref_m, rtol=2e-5)
    np.testing.assert_array_equal(gth.cpu().numpy(), project(mom).cpu().numpy())
