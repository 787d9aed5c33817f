"""Tessellation / basis checks (CPU).  For zero_boundary=True the reference's
basis is the column-normalised nodal hat-function map (tesselation.py:216-307);
it is pinned here by the published dimensions (d = 2210 at 24x24,
docs/index.html:194; d = 49 for [50]), by the constraints it must satisfy
(continuity across every shared face, zero velocity on the boundary, L B = 0,
unit columns) and by an independent restatement of the column order (active
vertices in first-seen order over the cells, 2 DOFs each), as the reference's
WebGPU port states it (docs/src/tessellation2d.js:8-13,85-102)."""
import pickle

import numpy as np
import pytest
import scipy.sparse as sp

from cpab.core.tesselation import Tesselation1D, Tesselation2D, Tesselation3D
from cpab.core.utility import load_obj, save_obj


@pytest.mark.parametrize("tess,d", [([50], 49), ([20, 20], 1522), ([30, 30], 3482),
                                    ([16, 16], 962), ([24, 24], 2210), ([10, 10, 10], 2187),
                                    ([5], 4), ([2, 3], 2 * (1 * 2 + 6)), ([3, 3, 3], 3 * 8)])
def test_dimensions(tess, d):
    cls = {1: Tesselation1D, 2: Tesselation2D, 3: Tesselation3D}[len(tess)]
    n = len(tess)
    T = cls(tess, [0] * n, [1] * n, True, False, None)
    assert T.B.shape == ({1: 2, 2: 6, 3: 12}[n] * T.nC, d)


def _tess(nc, zb=True, vp=False):
    n = len(nc)
    cls = {1: Tesselation1D, 2: Tesselation2D, 3: Tesselation3D}[n]
    return cls(nc, [0] * n, [1] * n, zb, vp, None)


@pytest.mark.parametrize("nc", [[6], [4, 3], [2, 3, 2]])
def test_field_continuous_and_zero_on_boundary(nc):
    T = _tess(nc)
    nd = len(nc)
    theta = np.random.default_rng(1).standard_normal(T.B.shape[1])
    A = (T.B @ theta).reshape(T.nC, nd, nd + 1)
    # continuity: both cells of every shared face agree at the face's vertices
    for (ci, cj), face in zip(T.shared_v_idx, T.shared_v):
        for v in face:
            np.testing.assert_allclose(A[ci] @ v, A[cj] @ v, atol=1e-12)
    # boundary vertices do not move
    for c in range(T.nC):
        for v in T.verts[c]:
            if ((v[:nd] == 0) | (v[:nd] == 1)).any():
                np.testing.assert_allclose(A[c] @ v, 0, atol=1e-12)
    np.testing.assert_allclose(np.asarray(abs(T.L @ T.B).max()), 0, atol=1e-10)


@pytest.mark.parametrize("nc", [[7], [3, 4], [2, 2, 3]])
def test_columns_unit_norm(nc):
    T = _tess(nc)
    norms = np.sqrt(np.asarray(T.B.power(2).sum(axis=0))).ravel()
    np.testing.assert_allclose(norms, 1.0, rtol=1e-12)


def _nodal_2d_closed_form(nx, ny):
    """Independent restatement for 2D: velocity u at active vertex a enters cell
    c's affine map through the hat function of that vertex; columns 2a+k in
    first-seen vertex order over (centre, corner, corner) of each triangle."""
    Vx, Vy = np.linspace(0, 1, nx + 1), np.linspace(0, 1, ny + 1)
    order, rows = {}, []
    for i in range(ny):
        for j in range(nx):
            ce = ((Vx[j] + Vx[j + 1]) / 2, (Vy[i] + Vy[i + 1]) / 2)
            ul, ur, ll, lr = (Vx[j], Vy[i]), (Vx[j + 1], Vy[i]), (Vx[j], Vy[i + 1]), (Vx[j + 1], Vy[i + 1])
            for tri in ((ce, ul, ur), (ce, ur, lr), (ce, lr, ll), (ce, ll, ul)):
                rows.append(tri)
                for v in tri:
                    if v not in order:
                        order[v] = None
    active = [v for v in order if not (v[0] in (0.0, 1.0) or v[1] in (0.0, 1.0))]
    idx = {v: a for a, v in enumerate(active)}
    N = np.zeros((6 * len(rows), 2 * len(active)))
    for c, tri in enumerate(rows):
        X = np.array([[v[0], v[1], 1.0] for v in tri])
        W = np.linalg.inv(X.T)  # row l: affine coefficients of vertex l's hat function
        for l, v in enumerate(tri):
            if v in idx:
                for k in range(2):
                    N[6 * c + 3 * k: 6 * c + 3 * k + 3, 2 * idx[v] + k] = W[l]
    return N / np.linalg.norm(N, axis=0)


@pytest.mark.parametrize("nc", [[2, 2], [4, 3], [5, 5]])
def test_2d_basis_matches_closed_form_order(nc):
    T = _tess(nc)
    np.testing.assert_allclose(T.B.toarray(), _nodal_2d_closed_form(*nc), atol=1e-12)


def test_verts_order_matches_lookup_convention():
    # cell 4*(jx + iy*nx) + t, t = 0 top, 1 right, 2 bottom, 3 left, centre first
    T = _tess([3, 2])
    c = 4 * (1 + 1 * 3) + 1
    np.testing.assert_allclose(T.verts[c], [[0.5, 0.75, 1], [2 / 3, 0.5, 1], [2 / 3, 1, 1]])
    T3 = _tess([2, 2, 2])
    assert T3.verts.shape == (40, 4, 4)
    # the five tetrahedra of a cube tile it: volumes sum to the cube volume
    vol = sum(abs(np.linalg.det(T3.verts[c][1:, :3] - T3.verts[c][0, :3])) / 6 for c in range(5))
    assert abs(vol - 1 / 8) < 1e-12


@pytest.mark.parametrize("nc,zb,vp", [([4, 3], False, False), ([4, 3], True, True),
                                      ([5], False, True), ([2, 2, 2], False, False)])
def test_general_basis_satisfies_constraints(nc, zb, vp):
    # SVD branch (zero_boundary=False or volume preservation): the null-space
    # basis is unique only up to rotation, so here only its defining properties
    # are checked; the exact columns are pinned by the reference-generated
    # fixtures in test_basis_golden.py.
    T = _tess(nc, zb, vp)
    assert T.B.shape[1] > 0
    assert abs(T.L @ T.B).max() < 1e-5
    norms = np.sqrt(np.asarray(T.B.power(2).sum(axis=0))).ravel()
    np.testing.assert_allclose(norms, 1.0, rtol=1e-10)
    if vp:
        nd = len(nc)
        A = (T.B @ np.random.default_rng(0).standard_normal(T.B.shape[1])).reshape(T.nC, nd, nd + 1)
        np.testing.assert_allclose(np.trace(A[:, :, :nd], axis1=1, axis2=2), 0, atol=1e-6)


def test_cache_roundtrip_and_name(tmp_path):
    d = str(tmp_path) + "/"
    T1 = Tesselation2D([3, 2], [0, 0], [1, 1], True, False, d)
    name = d + "cpab_basis_dim2_tess3_2_vo0_zb1_vp0_nodal_v2.pkl"
    assert (tmp_path / "cpab_basis_dim2_tess3_2_vo0_zb1_vp0_nodal_v2.pkl").exists()
    T2 = Tesselation2D([3, 2], [0, 0], [1, 1], True, False, d)
    assert (T1.B != T2.B).nnz == 0
    assert name.endswith(".pkl")


class _Call:
    """Pickles as a call of fn(*args) when loaded."""

    def __init__(self, fn, *args):
        self.fn, self.args = fn, args

    def __reduce__(self):
        return (self.fn, self.args)


@pytest.mark.parametrize("fn,args", [
    (print, ("pwned",)),
    # public callables of numpy itself: writing files, loading native code
    (np.savetxt, ("{out}", np.arange(3))),
    (np.save, ("{out}", np.arange(3))),
    (np.ctypeslib.load_library, ("libm", "/usr/lib")),
    (np.memmap, ("{out}",)),
    (np.load, ("{out}",)),
    # a scipy.sparse module function (only the matrix classes are allowed)
    (sp.save_npz, ("{out}", sp.csr_matrix(np.eye(2)))),
])
def test_cache_loader_refuses_code(tmp_path, fn, args):
    out = str(tmp_path / "written")
    args = tuple(a.format(out=out) if isinstance(a, str) else a for a in args)
    path = str(tmp_path / "evil")
    with open(path + ".pkl", "wb") as f:
        pickle.dump({"x": _Call(fn, *args)}, f)
    with pytest.raises(pickle.UnpicklingError):
        load_obj(path)
    assert not any(p.name.startswith("written") for p in tmp_path.iterdir())


def test_cache_loader_reads_arrays_and_sparse(tmp_path):
    path = str(tmp_path / "ok")
    obj = {"a": np.arange(3), "s": np.float64(2.5), "i": np.int64(7),
           "B": sp.csr_matrix(np.eye(3)), "C": sp.coo_matrix(np.eye(2)), "t": (1, [2.0], {"k": "v"})}
    save_obj(obj, path)
    back = load_obj(path)
    assert (back["a"] == np.arange(3)).all() and back["s"] == 2.5 and back["i"] == 7
    assert (back["B"] != obj["B"]).nnz == 0 and (back["C"].toarray() == np.eye(2)).all()
    assert back["t"] == (1, [2.0], {"k": "v"})
