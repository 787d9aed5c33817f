"""TEST INFRASTRUCTURE ONLY -- numpy front end of the C oracle (lib/liboracle.so).

The parity checker and the "reference-semantics CPU restatement" baseline.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it;
the product path (fg-cpab_amd/cpab) never imports it.

Every function takes / returns numpy arrays.  ``*_f32`` routines restate the
reference kernels op for op in float32; ``*_f64`` twins run the same scheme in
float64 to pin the mathematics (finite differences, closed forms).

How each function is pinned (tests/test_oracle.py unless noted; the reference
ships no tests or golden vectors for this path, and its CUDA cannot run here):
  cells               barycentric containment in the tessellation's cells;
                      boundary-projection rule for points outside (2D/3D)
  expm                scipy.linalg.expm (float64) at three norm ranges, incl.
                      the squaring branch; A = 0 gives I exactly
  affine, project     dense B @ theta and B^T @ M
  forward_trels       one uniform field in every cell: T steps = expm(A) p
  forward_midpoint    second-order convergence to the exact flow
  forward_closed_1d   scipy solve_ivp of the ODE; order preservation
  backward            float64 finite differences of the midpoint scheme
                      (1D/2D/3D); closed form at theta = 0; linearity in the seed
  adaptive substeps   (forward_trels / forward_midpoint / backward with
                      adaptive=True) one corrected step against an independent
                      float64 evaluation of p + (h/2)(A_c[p;1] + A_ce[q;1]) with a
                      different field per cell (1D/2D/3D); bit-identity with the
                      plain scheme on trajectories that never cross (and for the
                      backward at T = 1); the bound on the corrected endpoint's
                      offset for a cell-independent field
  interp_forward/     textbook bilinear; torch grid_sample (align_corners=True,
  interp_backward     border padding); finite differences
  (basis, host code)  fixtures written by the reference's tesselation.py
                      (tests/test_basis_golden.py)
No function is left "parity unpinned".  What stays unpinned is the exact
bits of the reference's own CUDA build (nvcc contraction choices, cuSPARSE
summation order, CUDA expf/logf), which no GPU here can produce.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.realpath(__file__))
LIB = os.path.join(_HERE, "lib", "liboracle.so")
_lib = None

_i, _l, _f, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.isfile(LIB):
            build()
        L = ctypes.CDLL(LIB)
        sig = {
            "orc_cells_f32": [_i, _l, _p, _i, _i, _i, _p],
            "orc_expm_f32": [_i, _l, _f, _p, _p],
            "orc_affine": [_l, _i, _i, _p, _p, _p, _p, _p],
            "orc_project": [_l, _i, _i, _p, _p, _p, _p, _p],
            "orc_forward_trels": [_i, _l, _l, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p],
            "orc_forward_midpoint": [_i, _l, _l, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p],
            "orc_backward": [_i, _l, _l, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p],
            "orc_forward_closed_1d": [_l, _l, _i, _i, _p, _p, _p],
            "orc_interp_forward": [_i, _l, _l, _p, _p, _p, _p, _p],
            "orc_interp_backward": [_i, _l, _l, _p, _p, _p, _p, _p, _p, _p],
        }
        for name, args in sig.items():
            for full in (name, name + "_f32", name + "_f64"):
                fn = getattr(L, full, None) if hasattr(L, full) else None
                if fn is not None:
                    fn.argtypes = args
                    fn.restype = None
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _suffix(dtype):
    return "_f64" if np.dtype(dtype) == np.float64 else "_f32"


def cells(ndim, points, nc):
    """Cell index of each point (points [ndim, n])."""
    pts = _c(points, np.float32)
    n = pts.shape[1]
    out = np.empty(n, np.int32)
    nx, ny, nz = (list(nc) + [1, 1])[:3]
    lib().orc_cells_f32(ndim, n, _ptr(pts), nx, ny, nz, _ptr(out))
    return out


def expm(ndim, As, dT):
    A = _c(As, np.float32)
    P = ndim * (ndim + 1)
    out = np.empty_like(A)
    lib().orc_expm_f32(ndim, A.size // P, ctypes.c_float(dT), _ptr(A), _ptr(out))
    return out


def affine(theta, B, dtype=np.float32):
    """As = B theta with fma in CSR column order.  B: scipy sparse [D, d]."""
    Bc = B.tocsr().astype(np.float64)
    Bc.sort_indices()
    th = _c(theta, dtype)
    n_theta, d = th.shape
    rows = Bc.shape[0]
    out = np.empty((n_theta, rows), dtype)
    getattr(lib(), "orc_affine" + _suffix(dtype))(
        n_theta, rows, d, _ptr(th), _ptr(_c(Bc.indptr, np.int32)), _ptr(_c(Bc.indices, np.int32)),
        _ptr(_c(Bc.data, dtype)), _ptr(out))
    return out


def project(moments, B, dtype=np.float32):
    """grad = B^T vec(M) with fma in CSC row order.  moments [n_theta, D]."""
    Bt = B.tocsc().astype(np.float64)
    Bt.sort_indices()
    M = _c(moments, dtype).reshape(moments.shape[0], -1)
    n_theta, D = M.shape
    d = Bt.shape[1]
    out = np.empty((n_theta, d), dtype)
    getattr(lib(), "orc_project" + _suffix(dtype))(
        n_theta, D, d, _ptr(M), _ptr(_c(Bt.indptr, np.int32)), _ptr(_c(Bt.indices, np.int32)),
        _ptr(_c(Bt.data, dtype)), _ptr(out))
    return out


def _geo(nc):
    return (list(nc) + [1, 1])[:3]


def _pts(points, n_theta, dtype):
    pts = _c(points, dtype)
    batched = int(pts.ndim == 3)
    return pts, batched, pts.shape[-1], pts.shape[-2]


def forward_trels(points, Trels, As, nc, T, adaptive=False, n_theta=None, return_cells=False,
                  dtype=np.float32, return_path=False):
    """Trels stepping (2D/3D forward).  Trels/As [n_theta, nC, ndim, ndim+1].
    return_path: also the position each step looks up, [n_theta, T, ndim, nP]."""
    Tr, A = _c(Trels, dtype), _c(As, dtype)
    n_theta = Tr.shape[0]
    pts, batched, nP, ndim = _pts(points, n_theta, dtype)
    out = np.empty((n_theta, ndim, nP), dtype)
    cl = np.empty((n_theta, nP, T), np.int32) if return_cells else None
    path = np.empty((n_theta, T, ndim, nP), dtype) if return_path else None
    nx, ny, nz = _geo(nc)
    getattr(lib(), "orc_forward_trels" + _suffix(dtype))(
        ndim, nP, n_theta, batched, T, nx, ny, nz, int(adaptive), _ptr(pts), _ptr(Tr), _ptr(A),
        _ptr(out), _ptr(cl), _ptr(path))
    res = (out,) + ((cl,) if return_cells else ()) + ((path,) if return_path else ())
    return res if len(res) > 1 else out


def forward_midpoint(points, As, nc, T, adaptive=False, return_cells=False, dtype=np.float32,
                     return_path=False):
    """Explicit-midpoint trajectory endpoint: the map the backward differentiates.
    return_path: also the position each step looks up, [n_theta, T, ndim, nP]."""
    A = _c(As, dtype)
    n_theta = A.shape[0]
    pts, batched, nP, ndim = _pts(points, n_theta, dtype)
    out = np.empty((n_theta, ndim, nP), dtype)
    cl = np.empty((n_theta, nP, T), np.int32) if return_cells else None
    path = np.empty((n_theta, T, ndim, nP), dtype) if return_path else None
    nx, ny, nz = _geo(nc)
    getattr(lib(), "orc_forward_midpoint" + _suffix(dtype))(
        ndim, nP, n_theta, batched, T, nx, ny, nz, int(adaptive), _ptr(pts), _ptr(A), _ptr(out),
        _ptr(cl), _ptr(path))
    res = (out,) + ((cl,) if return_cells else ()) + ((path,) if return_path else ())
    return res if len(res) > 1 else out


def backward(points, As, grad_out, nc, T, adaptive=False, dtype=np.float32):
    """Moments [n_theta, nC, ppc] (float64 accumulation) and grad_points [n_theta, ndim, nP]."""
    A = _c(As, dtype)
    n_theta, nC = A.shape[0], A.shape[1]
    pts, batched, nP, ndim = _pts(points, n_theta, dtype)
    g = _c(grad_out, dtype)
    P = ndim * (ndim + 1)
    mom = np.empty((n_theta, nC, P), np.float64)
    gp = np.empty((n_theta, ndim, nP), dtype)
    nx, ny, nz = _geo(nc)
    getattr(lib(), "orc_backward" + _suffix(dtype))(
        ndim, nP, n_theta, batched, T, nx, ny, nz, int(adaptive), _ptr(pts), _ptr(A), _ptr(g),
        _ptr(mom), _ptr(gp))
    return mom, gp


def forward_closed_1d(points, As, nc, dtype=np.float32):
    A = _c(As, dtype)
    n_theta = A.shape[0]
    pts, batched, nP, _ = _pts(points, n_theta, dtype)
    out = np.empty((n_theta, 1, nP), dtype)
    getattr(lib(), "orc_forward_closed_1d" + _suffix(dtype))(
        nP, n_theta, batched, int(nc[0]), _ptr(pts), _ptr(A), _ptr(out))
    return out


def interp_forward(ndim, data, grid, outsize, dtype=np.float32):
    d, g = _c(data, dtype), _c(grid, dtype)
    B, C = d.shape[:2]
    out = np.empty((B, C, *outsize), dtype)
    ins = _c(d.shape[2:], np.int64)
    outs = _c(outsize, np.int64)
    getattr(lib(), "orc_interp_forward" + _suffix(dtype))(
        ndim, B, C, _ptr(ins), _ptr(outs), _ptr(d), _ptr(g), _ptr(out))
    return out


def interp_backward(ndim, data, grid, outsize, grad_out, want_data=True, dtype=np.float32):
    d, g, go = _c(data, dtype), _c(grid, dtype), _c(grad_out, dtype)
    B, C = d.shape[:2]
    gg = np.empty_like(g)
    gd = np.empty_like(d) if want_data else None
    ins = _c(d.shape[2:], np.int64)
    outs = _c(outsize, np.int64)
    getattr(lib(), "orc_interp_backward" + _suffix(dtype))(
        ndim, B, C, _ptr(ins), _ptr(outs), _ptr(d), _ptr(g), _ptr(go), _ptr(gg), _ptr(gd))
    return gg, gd
