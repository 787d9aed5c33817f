"""The reference's ``cpab_gpu`` extension module, on ``libcpab_hip.so``.

The reference JIT-builds a pybind11 module ``cpab_gpu``
(``cpab/pytorch/transformer.py:9-21``) with five functions
(``cpab/pytorch/transformer_cuda.cpp:172-179``).  This module provides the same
five functions, with the same arguments, return shapes and zero-initialised
outputs, on top of the C ABI in ``include/cpab_hip.h``.  A code base that
keeps the reference's Python layer adopts the MI355X kernels by replacing
its ``cpab_gpu`` import with ``from . import cpab_gpu_hip as cpab_gpu``.

Conventions kept from the reference binding:
  - inputs are contiguous float32 GPU tensors (``CHECK_INPUT``,
    transformer_cuda.cpp:25-27);
  - ``broadcast`` = points are ``[batch, ndim, nP]`` with batch equal to the
    tables' batch (transformer_cuda.cpp:43,77,105,136);
  - 3D: ``ncz`` is inferred from nC as ``nC / (5 ncx ncy)``
    (transformer_cuda.cu:65-75);
  - shape and argument errors raise ``RuntimeError`` (the reference's
    ``AT_ASSERTM`` / ``TORCH_CHECK``).
Differences: work is enqueued on torch's current stream (the reference used the
legacy default stream), and a launch failure raises ``RuntimeError`` instead of
ending the process (transformer_cuda.cu:12-18).

The library path is ``$CPAB_HIP_LIB`` if set, else this package's in-tree
build (``cpab/lib/libcpab_hip.so``).
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.realpath(__file__))
_LIB_PATH = os.environ.get("CPAB_HIP_LIB") or os.path.join(_HERE, "..", "lib", "libcpab_hip.so")
if not os.path.isfile(_LIB_PATH):
    raise RuntimeError(f"libcpab_hip.so not found at {_LIB_PATH}; build it with "
                       f"`make -C fg-cpab_amd/csrc` or set CPAB_HIP_LIB")
_lib = ctypes.CDLL(_LIB_PATH)
_i, _l, _f, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_lib.cpab_last_error_string.restype = ctypes.c_char_p
_lib.cpab_expm.argtypes = [_i, _l, _f, _p, _p, _p]
_lib.cpab_forward.argtypes = [_i, _l, _l, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p]
_lib.cpab_forward_1d_closed_form.argtypes = [_l, _l, _i, _i, _p, _p, _p, _p]
_lib.cpab_backward_workspace_size.restype = _l
_lib.cpab_backward_workspace_size.argtypes = [_i, _l, _l, _i]
_lib.cpab_backward.argtypes = [_i, _l, _l, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _l, _p]


def _ok(rc):
    if rc != 0:
        raise RuntimeError(_lib.cpab_last_error_string().decode(errors="replace"))


def _check_input(name, t):
    if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
        raise RuntimeError(f"{name} must be a contiguous float32 GPU tensor")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ncz(ndim, nC, ncx, ncy):
    """ncz of a 3D tessellation from its cell count (transformer_cuda.cu:65-75)."""
    if ndim != 3:
        return 1
    per_z = 5 * ncx * ncy
    if per_z <= 0:
        raise RuntimeError(f"Invalid ncx/ncy for 3D: {ncx} x {ncy}")
    if nC % per_z != 0:
        raise RuntimeError(f"Could not infer ncz from nC={nC}, ncx={ncx}, ncy={ncy} "
                           f"(expected nC to be divisible by 5*ncx*ncy={per_z}).")
    return nC // per_z


def _broadcast(points, batch):
    return int(points.dim() == 3 and points.shape[0] == batch)


def expm(As_in, dT):                                          # transformer_cuda.cpp:159-170
    """expm(dT * [A; 0]) of each [ndim, ndim+1] block: As_in [n, ndim, ndim+1]."""
    _check_input("As_in", As_in)
    ndim = As_in.shape[1]
    if ndim not in (1, 2, 3):
        raise RuntimeError("As_in must have ndim=1,2,3 in dim 1")
    if As_in.dim() != 3 or As_in.shape[2] != ndim + 1:
        raise RuntimeError("As_in must be affine with shape [n, ndim, ndim+1]")
    out = torch.zeros_like(As_in)
    _ok(_lib.cpab_expm(ndim, As_in.shape[0], float(dT), _ptr(As_in), _ptr(out), _stream(As_in)))
    return out


def forward(points_in, trels_in, As_in, nstepsolver, ncx, ncy, adaptive_substeps):  # cpp:32-61
    """Transformed points [batch, ndim, nP]; 1D dispatches to the closed form."""
    for name, t in (("points_in", points_in), ("trels_in", trels_in), ("As_in", As_in)):
        _check_input(name, t)
    batch = trels_in.shape[0]
    broadcast = _broadcast(points_in, batch)
    ndim = points_in.shape[1] if broadcast else points_in.shape[0]
    nP = points_in.shape[-1]
    if As_in.shape[0] != batch:
        raise RuntimeError("As_in batch dimension mismatch")
    for k, what in ((1, "nC"), (2, "ndim"), (3, "affine")):
        if As_in.shape[k] != trels_in.shape[k]:
            raise RuntimeError(f"As_in {what} dimension mismatch")
    if adaptive_substeps not in (0, 1):
        raise RuntimeError("adaptive_substeps must be 0 or 1")
    out = torch.zeros((batch, ndim, nP), device=points_in.device)
    if ndim == 1:
        _ok(_lib.cpab_forward_1d_closed_form(nP, batch, broadcast, int(ncx), _ptr(points_in),
                                             _ptr(As_in), _ptr(out), _stream(points_in)))
        return out
    nC = As_in.shape[1]
    ncz = _ncz(ndim, nC, ncx, ncy)
    _ok(_lib.cpab_forward(ndim, nP, batch, broadcast, int(nstepsolver), int(ncx), int(ncy), ncz,
                          int(adaptive_substeps), _ptr(points_in), _ptr(trels_in), _ptr(As_in),
                          _ptr(out), _stream(points_in)))
    return out


def forward_1d_closed_form(points_in, As_in, ncx):                # transformer_cuda.cpp:66-85
    """1D closed-form flow: [batch, 1, nP]."""
    _check_input("points_in", points_in)
    _check_input("As_in", As_in)
    if As_in.dim() != 4:
        raise RuntimeError("As_in must have shape [batch, nC, 1, 2]")
    if As_in.shape[2] != 1 or As_in.shape[3] != 2:
        raise RuntimeError("As_in must have affine 1D shape [batch, nC, 1, 2]")
    batch = As_in.shape[0]
    broadcast = _broadcast(points_in, batch)
    ndim = points_in.shape[1] if broadcast else points_in.shape[0]
    if ndim != 1:
        raise RuntimeError("points_in must be 1D for forward_1d_closed_form")
    nP = points_in.shape[-1]
    out = torch.zeros((batch, 1, nP), device=points_in.device)
    _ok(_lib.cpab_forward_1d_closed_form(nP, batch, broadcast, int(ncx), _ptr(points_in),
                                         _ptr(As_in), _ptr(out), _stream(points_in)))
    return out


def _backward(points_in, As_in, grad_output_in, nstepsolver, ncx, ncy, adaptive_substeps,
              want_points):
    for name, t in (("points_in", points_in), ("As_in", As_in), ("grad_output_in", grad_output_in)):
        _check_input(name, t)
    if adaptive_substeps not in (0, 1):
        raise RuntimeError("adaptive_substeps must be 0 or 1")
    n_theta, nC, ndim = As_in.shape[0], As_in.shape[1], As_in.shape[2]
    broadcast = _broadcast(points_in, n_theta)
    nP = points_in.shape[-1]
    ncz = _ncz(ndim, nC, ncx, ncy)
    dev = points_in.device
    moments = torch.zeros((n_theta, nC, ndim * (ndim + 1)), device=dev)
    gp = torch.zeros((n_theta, ndim, nP), device=dev) if want_points else None
    nbytes = _lib.cpab_backward_workspace_size(ndim, nP, n_theta, nC)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _ok(_lib.cpab_backward(ndim, nP, n_theta, broadcast, int(nstepsolver), int(ncx), int(ncy), ncz,
                           int(adaptive_substeps), _ptr(points_in), _ptr(As_in),
                           _ptr(grad_output_in), _ptr(moments), _ptr(gp), _ptr(ws), nbytes,
                           _stream(points_in)))
    return moments, gp


def backward_moments(points_in, As_in, grad_output_in, nstepsolver, ncx, ncy,
                     adaptive_substeps):                            # transformer_cuda.cpp:92-116
    """Cell moments [n_theta, nC, ndim*(ndim+1)]."""
    return _backward(points_in, As_in, grad_output_in, nstepsolver, ncx, ncy, adaptive_substeps,
                     False)[0]


def backward_moments_and_points(points_in, As_in, grad_output_in, nstepsolver, ncx, ncy,
                                adaptive_substeps):                 # transformer_cuda.cpp:122-153
    """[moments, grad_points [n_theta, ndim, nP]]."""
    return list(_backward(points_in, As_in, grad_output_in, nstepsolver, ncx, ncy,
                          adaptive_substeps, True))
