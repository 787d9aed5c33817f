"""ctypes binding of ``libcpab_hip.so`` (declared in ``include/cpab_hip.h``).

The library is built in-tree (``make -C fg-cpab_amd/csrc``) into
``cpab/lib/libcpab_hip.so``.  There is no fallback: if the library is missing
or a call fails, a ``RuntimeError`` carrying the library's own message is
raised, mirroring the ``RuntimeError`` the reference's TORCH_CHECKs produce
(``cpab/pytorch/transformer_cuda.cpp:25-27``).
"""
import contextlib
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.realpath(__file__))
LIB_PATH = os.path.realpath(os.path.join(_HERE, "..", "lib", "libcpab_hip.so"))

_lock = threading.Lock()
_lib = None
_load_error = None

_c_int, _c_i64, _c_f32, _c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); must match include/cpab_hip.h
_SIGNATURES = {
    "cpab_last_error_string": (ctypes.c_char_p, []),
    "cpab_abi_version": (_c_int, []),
    "cpab_affine": (_c_int, [_c_int, _c_i64, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "cpab_expm": (_c_int, [_c_int, _c_i64, _c_f32, _c_vp, _c_vp, _c_vp]),
    "cpab_affine_expm": (_c_int, [_c_int, _c_i64, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                  _c_f32, _c_vp, _c_vp, _c_vp]),
    "cpab_forward": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int,
                              _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "cpab_forward_1d_closed_form": (_c_int, [_c_i64, _c_i64, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                                             _c_vp]),
    "cpab_trace_cells": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "cpab_backward_workspace_size": (_c_i64, [_c_int, _c_i64, _c_i64, _c_int]),
    "cpab_backward": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int,
                               _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_vp]),
    "cpab_backward_project": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp,
                                       _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_vp]),
    "cpab_backward_noalloc": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "cpab_chain_forward": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                    _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                    _c_vp]),
    "cpab_chain_backward_workspace_size": (_c_i64, [_c_int, _c_i64, _c_i64, _c_int, _c_int]),
    "cpab_chain_backward": (_c_int, [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                     _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_int,
                                     _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64,
                                     _c_vp]),
    "cpab_transform_data_forward": (_c_int, [_c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_int, _c_int,
                                             _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                             _c_vp, _c_vp, _c_vp, _c_vp]),
    "cpab_transform_data_backward_workspace_size": (_c_i64, [_c_int, _c_i64, _c_vp, _c_int]),
    "cpab_transform_data_backward_data_workspace_size": (_c_i64, [_c_int, _c_i64, _c_i64, _c_vp]),
    "cpab_transform_data_backward": (_c_int, [_c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_int, _c_int,
                                              _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                              _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                              _c_vp, _c_vp, _c_vp, _c_i64, _c_vp]),
    "cpab_project": (_c_int, [_c_i64, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "cpab_sum_batch": (_c_int, [_c_i64, _c_i64, _c_vp, _c_vp, _c_vp]),
    "cpab_interp_forward": (_c_int, [_c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                     _c_vp]),
    "cpab_set_deterministic": (None, [_c_int]),
    "cpab_deterministic": (_c_int, []),
    "cpab_profile_enable": (None, [_c_int]),
    "cpab_profile_read": (_c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(_c_i64)]),
    "cpab_interp_backward": (_c_int, [_c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                      _c_vp, _c_vp, _c_vp]),
    "cpab_interp_backward_workspace_size": (_c_i64, [_c_int, _c_i64, _c_i64, _c_vp]),
    "cpab_interp_backward_ws": (_c_int, [_c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                         _c_vp, _c_vp, _c_vp, _c_i64, _c_vp]),
}


def load_library(path=None):
    """Load (once) and return the ctypes handle; raises RuntimeError if absent."""
    global _lib, _load_error
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.isfile(p):
            _load_error = (f"libcpab_hip.so not found at {p}; build it with "
                           f"`make -C fg-cpab_amd/csrc` (or __graft_entry__.build())")
            raise RuntimeError(_load_error)
        lib = ctypes.CDLL(p)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def exported_symbols():
    return list(_SIGNATURES)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device):
    """Raw hipStream_t of torch's current stream on ``device`` (the launch stream)."""
    import torch
    idx = device.index if device.index is not None else torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return ctypes.c_void_p(raw(idx))
    return ctypes.c_void_p(torch.cuda.current_stream(idx).cuda_stream)


def _check(rc, what):
    if rc != 0:
        msg = _lib.cpab_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {msg}")


def _lengths(seq):
    arr = (ctypes.c_int64 * len(seq))(*[int(v) for v in seq])
    return arr


class Native:
    """Typed wrappers over the C ABI taking torch tensors (device pointers)."""

    def __init__(self):
        self.lib = load_library()

    def affine(self, ndim, theta, nC, row_ptr, col_idx, vals, As):
        _check(self.lib.cpab_affine(ndim, theta.shape[0], nC, theta.shape[1], _ptr(theta),
                                    _ptr(row_ptr), _ptr(col_idx), _ptr(vals), _ptr(As),
                                    _stream(theta.device)), "cpab_affine")

    def affine_expm(self, ndim, theta, nC, row_ptr, col_idx, vals, dT, As, Trels):
        _check(self.lib.cpab_affine_expm(ndim, theta.shape[0], nC, theta.shape[1], _ptr(theta),
                                         _ptr(row_ptr), _ptr(col_idx), _ptr(vals), float(dT),
                                         _ptr(As), _ptr(Trels), _stream(theta.device)),
               "cpab_affine_expm")

    def expm(self, ndim, As, dT, Trels):
        n = As.numel() // (ndim * (ndim + 1))
        _check(self.lib.cpab_expm(ndim, n, float(dT), _ptr(As), _ptr(Trels),
                                  _stream(As.device)), "cpab_expm")

    def forward(self, ndim, points, batched, n_theta, nP, T, nc, adaptive, Trels, As, out):
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        _check(self.lib.cpab_forward(ndim, nP, n_theta, int(batched), int(T), ncx, ncy, ncz,
                                     int(adaptive), _ptr(points), _ptr(Trels), _ptr(As),
                                     _ptr(out), _stream(points.device)), "cpab_forward")

    def forward_1d_closed_form(self, points, batched, n_theta, nP, ncx, As, out):
        _check(self.lib.cpab_forward_1d_closed_form(nP, n_theta, int(batched), ncx, _ptr(points),
                                                    _ptr(As), _ptr(out), _stream(points.device)),
               "cpab_forward_1d_closed_form")

    def trace_cells(self, ndim, points, batched, n_theta, nP, T, nc, adaptive, Trels, As, cells):
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        _check(self.lib.cpab_trace_cells(ndim, nP, n_theta, int(batched), int(T), ncx, ncy, ncz,
                                         int(adaptive), _ptr(points), _ptr(Trels), _ptr(As),
                                         _ptr(cells), _stream(points.device)), "cpab_trace_cells")

    @contextlib.contextmanager
    def deterministic(self, on):
        """Within the block, this thread's backward entry points (and their
        workspace sizes) use the deterministic two-pass reduction when ``on``:
        bit-identical moments, theta gradients and grad_data from run to run.
        The previous setting is restored on exit."""
        prev = int(self.lib.cpab_deterministic())
        self.lib.cpab_set_deterministic(1 if on else 0)
        try:
            yield
        finally:
            self.lib.cpab_set_deterministic(prev)

    def backward_workspace_size(self, ndim, nP, n_theta, nC):
        return int(self.lib.cpab_backward_workspace_size(ndim, nP, n_theta, nC))

    def backward(self, ndim, points, batched, n_theta, nP, T, nc, adaptive, As, grad_out,
                 moments, grad_points, workspace):
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        _check(self.lib.cpab_backward(ndim, nP, n_theta, int(batched), int(T), ncx, ncy, ncz,
                                      int(adaptive), _ptr(points), _ptr(As), _ptr(grad_out),
                                      _ptr(moments), _ptr(grad_points), _ptr(workspace), wbytes,
                                      _stream(points.device)), "cpab_backward")

    def backward_project(self, ndim, points, batched, n_theta, nP, T, nc, adaptive, As, grad_out,
                         tab, moments, grad_theta, grad_points, workspace):
        """cpab_backward and the projection onto the basis (tab: basis_tables)
        in one launch."""
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        _check(self.lib.cpab_backward_project(
            ndim, nP, n_theta, int(batched), int(T), ncx, ncy, ncz, int(adaptive), _ptr(points),
            _ptr(As), _ptr(grad_out), tab["d"], _ptr(tab["col_ptr"]), _ptr(tab["row_idx"]),
            _ptr(tab["vals_t"]), _ptr(moments), _ptr(grad_theta), _ptr(grad_points),
            _ptr(workspace), wbytes, _stream(points.device)), "cpab_backward_project")

    def backward_noalloc(self, ndim, points, batched, n_theta, nP, T, nc, adaptive, As, grad_out,
                         moments, grad_points):
        """cpab_backward without a caller workspace (the library's per-GPU
        scratch array; calls on one GPU must not overlap)."""
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        _check(self.lib.cpab_backward_noalloc(ndim, nP, n_theta, int(batched), int(T), ncx, ncy,
                                              ncz, int(adaptive), _ptr(points), _ptr(As),
                                              _ptr(grad_out), _ptr(moments), _ptr(grad_points),
                                              _stream(points.device)), "cpab_backward_noalloc")

    def chain_forward(self, ndim, points, batched, n_batch, n_stages, nP, T, nc, adaptive, Trels,
                      As, out, stage_points):
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        _check(self.lib.cpab_chain_forward(ndim, nP, n_batch, int(batched), n_stages, int(T), ncx,
                                           ncy, ncz, int(adaptive), _ptr(points), _ptr(Trels),
                                           _ptr(As), _ptr(out), _ptr(stage_points),
                                           _stream(points.device)), "cpab_chain_forward")

    def chain_backward_workspace_size(self, ndim, nP, n_batch, n_stages, nC):
        return int(self.lib.cpab_chain_backward_workspace_size(ndim, nP, n_batch, n_stages, nC))

    def chain_backward(self, ndim, points, batched, n_batch, n_stages, nP, T, nc, adaptive,
                       stage_points, As, grad_out, moments, grad_points, workspace, tab=None,
                       grad_theta=None):
        """tab (basis_tables) and grad_theta [n_stages * n_batch, d]: also
        project every row's moments onto the basis."""
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        proj = tab is not None and grad_theta is not None
        _check(self.lib.cpab_chain_backward(
            ndim, nP, n_batch, int(batched), n_stages, int(T), ncx, ncy, ncz, int(adaptive),
            _ptr(points), _ptr(stage_points), _ptr(As), _ptr(grad_out),
            tab["d"] if proj else 0, _ptr(tab["col_ptr"]) if proj else None,
            _ptr(tab["row_idx"]) if proj else None, _ptr(tab["vals_t"]) if proj else None,
            _ptr(moments), _ptr(grad_theta) if proj else None, _ptr(grad_points),
            _ptr(workspace), wbytes, _stream(points.device)), "cpab_chain_backward")

    def transform_data_forward(self, ndim, data, axes, outsize, T, nc, adaptive, Trels, As, out,
                               final_points, seed_grad=None):
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        _check(self.lib.cpab_transform_data_forward(
            ndim, data.shape[0], data.shape[1], _lengths(data.shape[2:]), _lengths(outsize),
            int(T), ncx, ncy, ncz, int(adaptive), _ptr(axes), _ptr(Trels), _ptr(As), _ptr(data),
            _ptr(out), _ptr(final_points), _ptr(seed_grad), _stream(data.device)),
            "cpab_transform_data_forward")

    def transform_data_backward_workspace_size(self, ndim, n_batch, outsize, nC):
        return int(self.lib.cpab_transform_data_backward_workspace_size(
            ndim, n_batch, _lengths(outsize), nC))

    def transform_data_backward_data_workspace_size(self, ndim, data):
        """Extra workspace bytes for grad_data in this thread's current mode
        (0 unless deterministic)."""
        return int(self.lib.cpab_transform_data_backward_data_workspace_size(
            ndim, data.shape[0], data.shape[1], _lengths(data.shape[2:])))

    def transform_data_backward(self, ndim, data, axes, outsize, T, nc, adaptive, final_points,
                                As, grad_out, moments, grad_data, workspace, tab=None,
                                grad_theta=None, seed_grad=None):
        """tab (basis_tables) and grad_theta [n_batch, d]: also project the
        moments onto the basis.  seed_grad: the forward's (one channel)."""
        ncx, ncy, ncz = (list(nc) + [1, 1])[:3]
        wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        proj = tab is not None and grad_theta is not None
        _check(self.lib.cpab_transform_data_backward(
            ndim, data.shape[0], data.shape[1], _lengths(data.shape[2:]), _lengths(outsize),
            int(T), ncx, ncy, ncz, int(adaptive), _ptr(axes), _ptr(final_points), _ptr(seed_grad),
            _ptr(As), _ptr(data), _ptr(grad_out), tab["d"] if proj else 0,
            _ptr(tab["col_ptr"]) if proj else None, _ptr(tab["row_idx"]) if proj else None,
            _ptr(tab["vals_t"]) if proj else None, _ptr(moments),
            _ptr(grad_theta) if proj else None, _ptr(grad_data), _ptr(workspace), wbytes,
            _stream(data.device)), "cpab_transform_data_backward")

    def project(self, moments, D, d, col_ptr, row_idx, vals, grad_theta):
        _check(self.lib.cpab_project(moments.shape[0], D, d, _ptr(moments), _ptr(col_ptr),
                                     _ptr(row_idx), _ptr(vals), _ptr(grad_theta),
                                     _stream(moments.device)), "cpab_project")

    def sum_batch(self, src, dst):
        n_theta = src.shape[0]
        _check(self.lib.cpab_sum_batch(n_theta, dst.numel(), _ptr(src), _ptr(dst),
                                       _stream(dst.device)), "cpab_sum_batch")

    def interp_forward(self, ndim, data, grid, outsize, out):
        _check(self.lib.cpab_interp_forward(ndim, data.shape[0], data.shape[1],
                                            _lengths(data.shape[2:]), _lengths(outsize),
                                            _ptr(data), _ptr(grid), _ptr(out),
                                            _stream(data.device)), "cpab_interp_forward")

    def interp_backward_workspace_size(self, ndim, data):
        """Workspace bytes of interp_backward_ws's grad_data in this thread's
        current mode (0 unless deterministic)."""
        return int(self.lib.cpab_interp_backward_workspace_size(
            ndim, data.shape[0], data.shape[1], _lengths(data.shape[2:])))

    def interp_backward_ws(self, ndim, data, grid, outsize, grad_out, grad_grid, grad_data,
                           workspace):
        wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        _check(self.lib.cpab_interp_backward_ws(ndim, data.shape[0], data.shape[1],
                                                _lengths(data.shape[2:]), _lengths(outsize),
                                                _ptr(data), _ptr(grid), _ptr(grad_out),
                                                _ptr(grad_grid), _ptr(grad_data), _ptr(workspace),
                                                wbytes, _stream(data.device)),
               "cpab_interp_backward_ws")

    def interp_backward(self, ndim, data, grid, outsize, grad_out, grad_grid, grad_data):
        _check(self.lib.cpab_interp_backward(ndim, data.shape[0], data.shape[1],
                                             _lengths(data.shape[2:]), _lengths(outsize),
                                             _ptr(data), _ptr(grid), _ptr(grad_out),
                                             _ptr(grad_grid), _ptr(grad_data),
                                             _stream(data.device)), "cpab_interp_backward")


def profile_enable(on=True):
    load_library().cpab_profile_enable(1 if on else 0)


def profile_read(kernel):
    """(total milliseconds, launches) recorded for ``kernel`` since the last read."""
    lib = load_library()
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    if lib.cpab_profile_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)) != 0:
        raise RuntimeError(lib.cpab_last_error_string().decode(errors="replace"))
    return ms.value, n.value


_native = None


def native():
    """Process-wide Native instance (loads the library on first use)."""
    global _native
    if _native is None:
        _native = Native()
    return _native
