"""Autograd entry point of the CPAB transform on MI355X.

Same interface as the reference's ``cpab/pytorch/transformer.py``:
``CPAB_transformer(points, theta, params, compute_points_grad=False)`` returns
the integrated points ``[n_theta, ndim, nP]`` and differentiates w.r.t. theta
(and the points when asked).  Every numeric step runs in the HIP library
(``libcpab_hip.so``) through its C ABI:

  forward   A = B theta and expm(A/T) in one launch (cpab_affine_expm) ->
            integrate (cpab_forward), or A = B theta (cpab_affine) and the 1D
            closed form                                 (transformer.py:72-126)
  backward  fused replay + adjoint + moments, and dtheta = B^T M, in one
            launch (cpab_backward_project) [-> sum over theta for shared points]
                                                        (transformer.py:128-168)

``CPAB_chain_transformer`` runs a whole chain of stages (the Python loop of
``Cpab.transform_grid_chain``, cpab/cpab.py:237-280) as one forward launch
(cpab_chain_forward) and one backward launch (cpab_chain_backward).

``CPAB_transform_data`` is ``Cpab.transform_data`` (transform_grid of the
meshgrid, then interpolate; cpab/cpab.py:295-309) as one forward launch
(cpab_transform_data_forward) and one backward launch
(cpab_transform_data_backward): the warped grid never leaves the kernels except
as the saved final points.
"""
import torch

from ._native import native

__all__ = ["CPAB_transformer", "CPAB_chain_transformer", "CPAB_transform_data"]


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


def _deterministic(params):
    """Whether the backward uses the deterministic two-pass reduction
    (``Cpab.set_solver_params(deterministic_grad=True)``)."""
    return bool(getattr(params, "deterministic_grad", False))


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
        nstepsolver = int(params.nstepsolver)
        adaptive = int(getattr(params, "adaptive_substeps", False))
        nc = [int(v) for v in params.nc]
        out = torch.empty((n_theta, ndim, nP), device=dev, dtype=torch.float32)
        if ndim == 1:
            lib.affine(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"], As)
            lib.forward_1d_closed_form(points_c, batched, n_theta, nP, nc[0], As, out)
        else:
            Trels = torch.empty_like(As)
            lib.affine_expm(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"],
                            1.0 / nstepsolver, As, Trels)
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
        want_points = ctx.compute_points_grad and ctx.needs_input_grad[0]
        gp = (torch.empty((n_theta, ndim, nP), device=dev, dtype=torch.float32)
              if want_points else None)
        tab = basis_tables(params, dev)
        grad_theta = torch.empty((n_theta, tab["d"]), device=dev, dtype=torch.float32)
        with lib.deterministic(_deterministic(params)):
            ws_bytes = lib.backward_workspace_size(ndim, nP, n_theta, nC)
            ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes > 0 else None
            # moments and their projection dtheta = B^T vec(M) in one launch
            lib.backward_project(ndim, points, ctx.batched, n_theta, nP, ctx.nstepsolver, ctx.nc,
                                 ctx.adaptive_substeps, As, grad, tab, moments, grad_theta, gp, ws)
        if want_points and points.dim() == 2:
            summed = torch.empty((ndim, nP), device=dev, dtype=torch.float32)
            lib.sum_batch(gp, summed)
            gp = summed
        return gp, grad_theta, None, None


def CPAB_chain_transformer(points, theta_stages, params):
    """Chain of CPAB transforms: stage s maps the output of stage s-1 with
    theta_stages[s]; equal, stage by stage, to chaining ``CPAB_transformer``
    (with compute_points_grad=True), as ``Cpab.transform_grid_chain`` does in
    the reference (cpab/cpab.py:270-278).

    Arguments:
        points: [ndim, n_points] (shared) or [n_batch, ndim, n_points]
        theta_stages: [n_stages, n_batch, d] (already scaled by dt if wanted)
    Returns:
        [n_batch, ndim, n_points]
    """
    assert points.is_cuda and theta_stages.is_cuda, "Only GPU tensors supported"
    assert params.ndim in (1, 2, 3), "GPU transformer supports 1D, 2D, and 3D"
    return _CPABChainFunction.apply(points, theta_stages, params)


class _CPABChainFunction(torch.autograd.Function):
    """All stages of a chain in one forward and one backward launch."""

    @staticmethod
    def forward(ctx, points, theta_stages, params):
        if theta_stages.dim() != 3:
            raise RuntimeError(f"theta_stages must be [n_stages, n_batch, d], got {tuple(theta_stages.shape)}")
        K, n_batch, d = theta_stages.shape
        batched, nP = _check_inputs(points, theta_stages[0], params)
        lib = native()
        dev = theta_stages.device
        ndim, nC = params.ndim, int(params.nC)
        tab = basis_tables(params, dev)
        theta_c = theta_stages.detach().reshape(K * n_batch, d).contiguous()
        points_c = points.detach().contiguous()

        As = torch.empty((K * n_batch, nC, ndim, ndim + 1), device=dev, dtype=torch.float32)
        nstepsolver = int(params.nstepsolver)
        adaptive = int(getattr(params, "adaptive_substeps", False))
        nc = [int(v) for v in params.nc]
        Trels = None
        if ndim > 1:
            Trels = torch.empty_like(As)
            lib.affine_expm(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"],
                            1.0 / nstepsolver, As, Trels)
        else:
            lib.affine(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"], As)
        grad_wanted = any(ctx.needs_input_grad[:2])
        stage_points = (torch.empty((K - 1, n_batch, ndim, nP), device=dev, dtype=torch.float32)
                        if grad_wanted and K > 1 else None)
        out = torch.empty((n_batch, ndim, nP), device=dev, dtype=torch.float32)
        lib.chain_forward(ndim, points_c, batched, n_batch, K, nP, nstepsolver, nc, adaptive,
                          Trels, As, out, stage_points)

        ctx.dims = (K, n_batch, nP)
        ctx.nstepsolver = nstepsolver
        ctx.nc = nc
        ctx.adaptive_substeps = adaptive
        ctx.params = params
        ctx.batched = batched
        ctx.save_for_backward(points_c, As, stage_points)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        points, As, stage_points = ctx.saved_tensors
        K, n_batch, nP = ctx.dims
        params = ctx.params
        lib = native()
        dev = As.device
        nC, ndim = As.shape[1], As.shape[2]
        ppc = ndim * (ndim + 1)
        grad = grad.detach().to(torch.float32).contiguous()

        moments = torch.empty((K * n_batch, nC, ppc), device=dev, dtype=torch.float32)
        want_points = ctx.needs_input_grad[0]
        gp = (torch.empty((n_batch, ndim, nP), device=dev, dtype=torch.float32)
              if want_points else None)
        tab = basis_tables(params, dev)
        grad_theta = torch.empty((K * n_batch, tab["d"]), device=dev, dtype=torch.float32)
        with lib.deterministic(_deterministic(params)):
            ws_bytes = lib.chain_backward_workspace_size(ndim, nP, n_batch, K, nC)
            ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes > 0 else None
            lib.chain_backward(ndim, points, ctx.batched, n_batch, K, nP, ctx.nstepsolver, ctx.nc,
                               ctx.adaptive_substeps, stage_points, As, grad, moments, gp, ws,
                               tab=tab, grad_theta=grad_theta)
        if want_points and points.dim() == 2:
            summed = torch.empty((ndim, nP), device=dev, dtype=torch.float32)
            lib.sum_batch(gp, summed)
            gp = summed
        return gp, grad_theta.view(K, n_batch, tab["d"]), None


def CPAB_transform_data(data, theta, axes, outsize, params):
    """``interpolate(data, CPAB_transformer(meshgrid, theta, params), outsize)``
    in one fused forward and one fused backward launch.

    Arguments:
        data: [n_batch, n_channels, *in_size]
        theta: [n_batch, d]
        axes: [sum(outsize)] the per-axis coordinates of the uniform grid, axis 0
            first (the ``torch.linspace`` vectors ``Cpab.uniform_meshgrid`` takes the
            Cartesian product of): the kernels look a pixel's start point up
            there instead of reading a meshgrid
        outsize: list of ndim output sizes
    Returns:
        [n_batch, n_channels, *outsize]
    """
    assert data.is_cuda and theta.is_cuda and axes.is_cuda, "Only GPU tensors supported"
    assert params.ndim in (1, 2, 3), "GPU transformer supports 1D, 2D, and 3D"
    return _CPABImageFunction.apply(data, theta, axes, [int(v) for v in outsize], params)


class _CPABImageFunction(torch.autograd.Function):
    """Fused transform_data: integrate the meshgrid and resample in one pass."""

    @staticmethod
    def forward(ctx, data, theta, axes, outsize, params):
        ndim, nC = params.ndim, int(params.nC)
        if data.dtype != torch.float32 or theta.dtype != torch.float32:
            raise RuntimeError("expected float32 data and theta")
        if data.dim() != ndim + 2:
            raise RuntimeError(f"data must be [n_batch, n_channels, *in_size] with {ndim} spatial axes")
        if theta.dim() != 2 or theta.shape[1] != params.d or theta.shape[0] != data.shape[0]:
            raise RuntimeError(f"theta must be [n_batch={data.shape[0]}, {params.d}], got {tuple(theta.shape)}")
        nP = 1
        for v in outsize:
            nP *= v
        if len(outsize) != ndim or tuple(axes.shape) != (sum(outsize),):
            raise RuntimeError("axes must be the [sum(outsize)] per-axis coordinates of the grid")
        lib = native()
        dev = theta.device
        n = theta.shape[0]
        tab = basis_tables(params, dev)
        data_c = data.detach().contiguous()
        axes_c = axes.detach().contiguous()
        As = torch.empty((n, nC, ndim, ndim + 1), device=dev, dtype=torch.float32)
        theta_c = theta.detach().contiguous()
        T = int(params.nstepsolver)
        adaptive = int(getattr(params, "adaptive_substeps", False))
        nc = [int(v) for v in params.nc]
        Trels = None
        if ndim > 1:
            Trels = torch.empty_like(As)
            lib.affine_expm(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"],
                            1.0 / T, As, Trels)
        else:
            lib.affine(ndim, theta_c, nC, tab["row_ptr"], tab["col_idx"], tab["vals"], As)
        # For the backward: with one channel and no grad_data the sample's
        # spatial gradient at each final point (the seed then needs no data
        # reads); the final points themselves when grad_data's scatter or
        # several channels need them.
        one = data.shape[1] == 1
        seed_grad = (torch.empty((n, ndim, nP), device=dev, dtype=torch.float32)
                     if ctx.needs_input_grad[1] and one and not ctx.needs_input_grad[0] else None)
        final = (torch.empty((n, ndim, nP), device=dev, dtype=torch.float32)
                 if ctx.needs_input_grad[0] or (ctx.needs_input_grad[1] and not one) else None)
        out = torch.empty((n, data.shape[1], *outsize), device=dev, dtype=torch.float32)
        lib.transform_data_forward(ndim, data_c, axes_c, outsize, T, nc, adaptive, Trels, As, out,
                                   final, seed_grad)
        ctx.outsize = list(outsize)
        ctx.T = T
        ctx.nc = nc
        ctx.adaptive = adaptive
        ctx.params = params
        ctx.save_for_backward(data_c, axes_c, final, seed_grad, As)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        data, axes, final, seed_grad, As = ctx.saved_tensors
        params = ctx.params
        lib = native()
        dev = As.device
        n, nC, ndim = As.shape[0], As.shape[1], As.shape[2]
        grad = grad.detach().to(torch.float32).contiguous()
        moments = torch.empty((n, nC, ndim * (ndim + 1)), device=dev, dtype=torch.float32)
        grad_data = torch.empty_like(data) if ctx.needs_input_grad[0] else None
        tab, grad_theta = None, None
        if ctx.needs_input_grad[1]:
            tab = basis_tables(params, dev)
            grad_theta = torch.empty((n, tab["d"]), device=dev, dtype=torch.float32)
        with lib.deterministic(_deterministic(params)):
            ws_bytes = lib.transform_data_backward_workspace_size(ndim, n, ctx.outsize, nC)
            if grad_data is not None:
                ws_bytes += lib.transform_data_backward_data_workspace_size(ndim, data)
            ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes > 0 else None
            lib.transform_data_backward(ndim, data, axes, ctx.outsize, ctx.T, ctx.nc,
                                        ctx.adaptive, final, As, grad, moments, grad_data, ws,
                                        tab=tab, grad_theta=grad_theta, seed_grad=seed_grad)
        return grad_data, grad_theta, None, None, None
