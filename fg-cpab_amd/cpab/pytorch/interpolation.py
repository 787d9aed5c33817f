"""``transform_data`` resampling on MI355X.

Same functions and semantics as the reference's
``cpab/pytorch/interpolation.py:3-159``: ``interpolate(ndim, data, grid,
outsize)`` samples ``data [B, C, *in_size]`` at ``grid [B, ndim,
prod(outsize)]`` (coordinate k scaled by ``in_size[k]-1`` and clamped to the
border) and returns ``[B, C, *outsize]``.  Forward and backward (w.r.t. the
grid, and w.r.t. the data when it requires grad) are HIP kernels behind the C
ABI; there is no torch or CPU fallback.  ``deterministic=True`` (an addition to
the reference's arguments; ``Cpab.interpolate`` passes the solver's
``deterministic_grad``) sums the data gradient as 64-bit integers, the same on
every run.
"""
import torch

from ._native import native

__all__ = ["interpolate", "interpolate1D", "interpolate2D", "interpolate3D"]


def interpolate(ndim, data, grid, outsize, deterministic=False):
    if ndim == 1:
        return interpolate1D(data, grid, outsize, deterministic)
    elif ndim == 2:
        return interpolate2D(data, grid, outsize, deterministic)
    elif ndim == 3:
        return interpolate3D(data, grid, outsize, deterministic)


def interpolate1D(data, grid, outsize, deterministic=False):
    return _Interp.apply(1, data, grid, tuple(int(v) for v in outsize), bool(deterministic))


def interpolate2D(data, grid, outsize, deterministic=False):
    return _Interp.apply(2, data, grid, tuple(int(v) for v in outsize), bool(deterministic))


def interpolate3D(data, grid, outsize, deterministic=False):
    return _Interp.apply(3, data, grid, tuple(int(v) for v in outsize), bool(deterministic))


def _check(ndim, data, grid, outsize):
    if not (data.is_cuda and grid.is_cuda):
        raise RuntimeError("interpolate: only GPU tensors are supported")
    if data.dtype != torch.float32 or grid.dtype != torch.float32:
        raise RuntimeError(f"interpolate: expected float32, got data {data.dtype}, grid {grid.dtype}")
    if data.dim() != ndim + 2 or len(outsize) != ndim:
        raise RuntimeError(f"interpolate: data must be [B, C, *{ndim} sizes] and outsize have "
                           f"{ndim} entries")
    nP = 1
    for v in outsize:
        nP *= v
    if grid.dim() != 3 or grid.shape[0] != data.shape[0] or grid.shape[1] != ndim \
            or grid.shape[2] != nP:
        raise RuntimeError(f"interpolate: grid must be [{data.shape[0]}, {ndim}, {nP}], "
                           f"got {tuple(grid.shape)}")


class _Interp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ndim, data, grid, outsize, deterministic=False):
        _check(ndim, data, grid, outsize)
        data_c = data.detach().contiguous()
        grid_c = grid.detach().contiguous()
        out = torch.empty((data.shape[0], data.shape[1], *outsize), device=data.device,
                          dtype=torch.float32)
        native().interp_forward(ndim, data_c, grid_c, outsize, out)
        ctx.ndim = ndim
        ctx.outsize = outsize
        ctx.deterministic = deterministic
        ctx.save_for_backward(data_c, grid_c)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        data, grid = ctx.saved_tensors
        need_data, need_grid = ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        if not (need_data or need_grid):
            return None, None, None, None, None
        g = grad_out.detach().to(torch.float32).contiguous()
        grad_grid = torch.empty_like(grid) if need_grid else None
        grad_data = torch.empty_like(data) if need_data else None
        lib = native()
        if ctx.deterministic and need_data:
            with lib.deterministic(True):
                nbytes = lib.interp_backward_workspace_size(ctx.ndim, data)
                ws = torch.empty(nbytes, device=data.device, dtype=torch.uint8)
                lib.interp_backward_ws(ctx.ndim, data, grid, ctx.outsize, g, grad_grid, grad_data,
                                       ws)
        else:
            lib.interp_backward(ctx.ndim, data, grid, ctx.outsize, g, grad_grid, grad_data)
        return None, grad_data, grad_grid, None, None
