"""Autograd entry point of the CPAB transform on MI355X.

Same interface as the reference's ``cpab/pytorch/transformer.py``:
``CPAB_transformer(points, theta, params, compute_points_grad=False)`` returns
the integrated points ``[n_theta, ndim, nP]`` and differentiates w.r.t. theta
(and the points when asked).  Every numeric step runs in the HIP library
(``libcpab_hip.so``) through its C ABI:

  forward   A = B theta (cpab_affine) -> expm(A/T) (cpab_expm) -> integrate
            (cpab_forward), or the 1D closed form      (transformer.py:72-126)
  backward  fused replay + adjoint + moments (cpab_backward) -> dtheta = B^T M
            (cpab_project) [-> sum over theta for shared points]
                                                        (transformer.py:128-168)
"""
import torch

from ._native import native

__all__ = ["CPAB_transformer"]


def CPAB_transformer(points, theta, params, compute_points_grad=False):
    """Transform points through the CPAB velocity field.

    Arguments:
        points: [ndim, n_points] (shared by all thetas) or [n_batch, ndim, n_points]
        theta: [n_batch, d]
        params: parameter object of a ``Cpab`` instance
        compute_points_grad: bool, also return d loss / d points in backward
    Returns:
        transformed points [n_batch, ndim, n_points]
    """
    assert points.is_cuda and theta.is_cuda, "Only GPU tensors supported"
    assert params.ndim in (1, 2, 3), "GPU transformer supports 1D, 2D, and 3D"
    assert type(compute_points_grad) == bool, "compute_points_grad must be bool"
    return _CPABFunction.apply(points, theta, params, compute_points_grad)


def basis_tables(params, device):
    """Device copies of B as CSR (for A = B theta) and CSC (for B^T M), float32.

    Cached on ``params`` per device.  Replaces the torch sparse COO copies the
    reference keeps in ``params.basis_gpu_sparse(_t)`` (transformer.py:47-66).
    """
    cache = params.__dict__.setdefault("_hip_basis_tables", {})
    key = str(device)
    t = cache.get(key)
    if t is not None:
        return t
    import numpy as np
    B = params.basis.tocsr().astype(np.float64)
    B.sort_indices()
    Bt = B.tocsc()
    Bt.sort_indices()

    def dev(a, dtype):
        return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)

    t = {
        "row_ptr": dev(B.indptr.astype(np.int32), torch.int32),
        "col_idx": dev(B.indices.astype(np.int32), torch.int32),
        "vals": dev(B.data.astype(np.float32), torch.float32),
        "col_ptr": dev(Bt.indptr.astype(np.int32), torch.int32),
        "row_idx": dev(Bt.indices.astype(np.int32), torch.int32),
        "vals_t": dev(Bt.data.astype(np.float32), torch.float32),
        "D": int(B.shape[0]),
        "d": int(B.shape[1]),
    }
    cache[key] = t
    return t


def _check_inputs(points, theta, params):
    if theta.dtype != torch.float32 or points.dtype != torch.float32:
        raise RuntimeError(f"expected float32 tensors, got points {points.dtype}, "
                           f"theta {theta.dtype}")
    if theta.dim() != 2 or theta.shape[1] != params.d:
        raise RuntimeError(f"theta must have shape [n_batch, {params.d}], got {tuple(theta.shape)}")
    if points.device != theta.device:
        raise RuntimeError("points and theta must be on the same device")
    n_theta = theta.shape[0]
    ndim = params.ndim
    batched = points.dim() == 3 and points.shape[0] == n_theta
    if points.dim() == 3 and not batched:
        raise RuntimeError(f"batched points have {points.shape[0]} entries but theta has {n_theta}")
    if points.dim() not in (2, 3) or points.shape[-2] != ndim:
        raise RuntimeError(f"points must be [{ndim}, nP] or [n_batch, {ndim}, nP], "
                           f"got {tuple(points.shape)}")
    return batched, int(points.shape[-1])


class _CPABFunction(torch.autograd.Function):
    """Analytical gradients by the discrete adjoint of the midpoint scheme."""

    @staticmethod
    def forward(ctx, points, theta, params, compute_points_grad=False):
        batched, nP = _check_inputs(points, theta, params)
        lib = native()
        dev = theta.device
        ndim, nC = params.ndim, int(params.nC)
        n_theta = theta.shape[0]
        tab = basis_tables(params, dev)
        theta_c = theta.detach().contiguous()
        points_c = points.detach().contiguous()

        As = torch.empty((n_theta, nC, ndim, ndim + 1), device=dev, dtype=torch.float32)
        lib.affine(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"], As)

        nstepsolver = int(params.nstepsolver)
        adaptive = int(getattr(params, "adaptive_substeps", False))
        nc = [int(v) for v in params.nc]
        out = torch.empty((n_theta, ndim, nP), device=dev, dtype=torch.float32)
        if ndim == 1:
            lib.forward_1d_closed_form(points_c, batched, n_theta, nP, nc[0], As, out)
        else:
            Trels = torch.empty_like(As)
            lib.expm(ndim, As, 1.0 / nstepsolver, Trels)
            lib.forward(ndim, points_c, batched, n_theta, nP, nstepsolver, nc, adaptive, Trels,
                        As, out)

        ctx.nstepsolver = nstepsolver
        ctx.nc = nc
        ctx.adaptive_substeps = adaptive
        ctx.compute_points_grad = compute_points_grad
        ctx.params = params
        ctx.batched = batched
        ctx.save_for_backward(points_c, As)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        points, As = ctx.saved_tensors
        params = ctx.params
        lib = native()
        dev = As.device
        n_theta, nC, ndim = As.shape[0], As.shape[1], As.shape[2]
        ppc = ndim * (ndim + 1)
        nP = points.shape[-1]
        grad = grad.detach().to(torch.float32).contiguous()

        moments = torch.empty((n_theta, nC, ppc), device=dev, dtype=torch.float32)
        ws_bytes = lib.backward_workspace_size(ndim, nP, n_theta, nC)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes > 0 else None
        want_points = ctx.compute_points_grad and ctx.needs_input_grad[0]
        gp = (torch.empty((n_theta, ndim, nP), device=dev, dtype=torch.float32)
              if want_points else None)
        lib.backward(ndim, points, ctx.batched, n_theta, nP, ctx.nstepsolver, ctx.nc,
                     ctx.adaptive_substeps, As, grad, moments, gp, ws)
        if want_points and points.dim() == 2:
            summed = torch.empty((ndim, nP), device=dev, dtype=torch.float32)
            lib.sum_batch(gp, summed)
            gp = summed

        tab = basis_tables(params, dev)
        grad_theta = torch.empty((n_theta, tab["d"]), device=dev, dtype=torch.float32)
        lib.project(moments.view(n_theta, -1), tab["D"], tab["d"], tab["col_ptr"],
                    tab["row_idx"], tab["vals_t"], grad_theta)
        return gp, grad_theta, None, None
