"""Public ``Cpab`` API (drop-in for the reference's ``cpab/cpab.py``).

Method names, arguments, defaults, shapes and assertion messages follow the
reference class (``cpab/cpab.py:11-333``).  The numeric work behind
``transform_grid``, ``transform_grid_chain``, ``interpolate`` and
``transform_data`` runs in HIP kernels on the GPU; the tessellation / basis is
built on the host once and cached in ``basis_files/``.
"""
import numpy as np
import torch

from .core.tesselation import Tesselation1D, Tesselation2D, Tesselation3D
from .core.utility import params, get_dir, create_dir
from .pytorch.transformer import CPAB_transformer as transformer
from .pytorch.transformer import CPAB_chain_transformer as chain_transformer
from .pytorch.transformer import CPAB_transform_data as transform_data_fused
from .pytorch.interpolation import interpolate

# GPU device constant (HIP devices are exposed as "cuda" by PyTorch-ROCm)
_DEVICE = torch.device("cuda")


class Cpab(object):
    """Continuous piecewise-affine transformations with an MI355X (HIP) backend.

    Arguments:
        tess_size: list of 1, 2, or 3 integers defining the number of cells
            per spatial dimension
        zero_boundary: bool, whether the boundary velocity is constrained to 0
        volume_perservation: bool, whether the transform is volume preserving
        override: bool, whether to rebuild and overwrite the cached basis
    """

    def __init__(self, tess_size, zero_boundary=True, volume_perservation=False,
                 override=False):
        self._check_input(tess_size, zero_boundary, volume_perservation, override)

        self.params = params()
        self.params.nc = tess_size
        self.params.ndim = len(tess_size)
        self.params.Ashape = [self.params.ndim, self.params.ndim + 1]
        self.params.valid_outside = not zero_boundary
        self.params.zero_boundary = zero_boundary
        self.params.volume_perservation = volume_perservation
        self.params.domain_max = [1] * self.params.ndim
        self.params.domain_min = [0] * self.params.ndim
        self.params.inc = [(self.params.domain_max[i] - self.params.domain_min[i])
                           / self.params.nc[i] for i in range(self.params.ndim)]
        self.params.nstepsolver = 50
        self.params.adaptive_substeps = False
        self.params.deterministic_grad = False

        self._dir = get_dir(__file__) + '/../basis_files/'
        create_dir(self._dir)

        if self.params.ndim == 1:
            self.params.nC = int(np.prod(self.params.nc))
            self.params.params_pr_cell = 2
            tesselation = Tesselation1D
        elif self.params.ndim == 2:
            self.params.nC = 4 * int(np.prod(self.params.nc))
            self.params.params_pr_cell = 6
            tesselation = Tesselation2D
        elif self.params.ndim == 3:
            self.params.nC = 5 * int(np.prod(self.params.nc))
            self.params.params_pr_cell = 12
            tesselation = Tesselation3D
        else:
            raise ValueError('Only 1D, 2D, and 3D tessellations are supported')

        self.tesselation = tesselation(self.params.nc, self.params.domain_min,
                                       self.params.domain_max, self.params.zero_boundary,
                                       self.params.volume_perservation, self._dir, override)

        self.params.constrain_mat = self.tesselation.L
        self.params.basis = self.tesselation.B
        self.params.D, self.params.d = self.params.basis.shape
        self.params.basis_gpu_sparse = None
        self.params.basis_gpu_sparse_t = None
        if torch.cuda.is_available():
            basis_sparse = self._get_basis_sparse_gpu(dtype=torch.float32, device=_DEVICE)
            self.params.basis_gpu_sparse_t = basis_sparse.transpose(0, 1).coalesce()

    def get_theta_dim(self):
        """Return the dimensionality of the transformation parameters."""
        return self.params.d

    def get_params(self):
        """Return the parameter container for the transformation."""
        return self.params

    def get_basis(self):
        """Return the basis matrix of the transformation."""
        return self.params.basis

    def _get_basis_sparse_gpu(self, dtype=torch.float32, device=_DEVICE):
        """Sparse COO copy of the basis on ``device`` (cached for float32 / device 0)."""
        B = self.params.basis_gpu_sparse
        if B is not None and B.dtype == dtype and B.device == device:
            return B
        coo = self.params.basis.tocoo()
        idx = torch.from_numpy(np.vstack((coo.row, coo.col)).astype(np.int64)).to(device=device)
        val = torch.from_numpy(coo.data).to(device=device, dtype=dtype)
        B = torch.sparse_coo_tensor(idx, val, size=self.params.basis.shape, device=device,
                                    dtype=dtype).coalesce()
        if device.type == "cuda" and device.index in (None, 0) and dtype == torch.float32:
            self.params.basis_gpu_sparse = B
            self.params.basis_gpu_sparse_t = B.transpose(0, 1).coalesce()
        return B

    def set_solver_params(self, nstepsolver=50, adaptive_substeps=False, *,
                          deterministic_grad=False):
        """Set parameters controlling the integration algorithm
        (``cpab/cpab.py:112-129``).

        Arguments:
            nstepsolver: int, number of integration steps
            adaptive_substeps: bool, Heun correction when a step crosses a cell
            deterministic_grad: bool (an addition to the reference's arguments),
                the GPU backward reduces its per-cell sums (and
                transform_data's data gradient) in 64-bit integers over two
                passes, so theta, point and data gradients are bit-identical
                from run to run on one device (the benchmark steps take about
                twice their default time)
        """
        assert nstepsolver > 0, 'nstepsolver must be a positive number'
        assert type(nstepsolver) == int, 'nstepsolver must be integer'
        assert type(adaptive_substeps) == bool, 'adaptive_substeps must be bool'
        assert type(deterministic_grad) == bool, 'deterministic_grad must be bool'
        self.params.nstepsolver = nstepsolver
        self.params.adaptive_substeps = adaptive_substeps
        self.params.deterministic_grad = deterministic_grad

    def uniform_meshgrid(self, n_points):
        """[ndim, prod(n_points)] grid over the domain, coordinate 0 varying fastest."""
        lin = self._linspaces(n_points)
        mesh = torch.meshgrid(lin[::-1], indexing='ij')
        return torch.cat([g.reshape(1, -1) for g in mesh[::-1]], dim=0)

    def sample_transformation(self, n_sample=1, mean=None, cov=None):
        """[n_sample, d] samples from N(mean, cov) (defaults: 0, I)."""
        d = self.params.d
        mean = torch.zeros(d, dtype=torch.float32, device=_DEVICE) if mean is None else mean
        cov = torch.eye(d, dtype=torch.float32, device=_DEVICE) if cov is None else cov
        return torch.distributions.MultivariateNormal(mean, cov).sample((n_sample,))

    def sample_transformation_with_prior(self, n_sample=1, mean=None, length_scale=0.1,
                                         output_variance=1):
        """Smooth samples: squared-exponential covariance between cell centres,
        mapped to theta space through the basis (``cpab/cpab.py:164-206``)."""
        centers = torch.tensor(self.tesselation.get_cell_centers(), dtype=torch.float32,
                               device=_DEVICE)
        norm = torch.sum(centers * centers, 1).reshape(-1, 1)
        dist = norm - 2 * centers.mm(centers.t()) + norm.t()
        ppc = self.params.params_pr_cell
        nC = self.params.nC
        # Block (i, j) of the [D, D] matrix: dist[i, j] on the diagonal,
        # 100 * max(dist) elsewhere.
        big = 100 * dist.max()
        eye = torch.eye(ppc, device=_DEVICE, dtype=torch.float32)
        cov_init = (dist[:, None, :, None] * eye[None, :, None, :]
                    + big * (1 - eye)[None, :, None, :]).reshape(nC * ppc, nC * ppc)
        cov_avees = output_variance ** 2 * torch.exp(-(cov_init / (2 * length_scale ** 2)))
        B_t = self._get_basis_sparse_gpu(dtype=torch.float32, device=_DEVICE).transpose(0, 1).coalesce()
        cov_avees_B = torch.sparse.mm(B_t, cov_avees.t()).t()
        cov_theta = torch.sparse.mm(B_t, cov_avees_B)
        return self.sample_transformation(n_sample, mean=mean, cov=cov_theta)

    def identity(self, n_sample=1, epsilon=0):
        """[n_sample, d] identity parameters (zeros + epsilon)."""
        assert epsilon >= 0, "epsilon need to be larger than 0"
        return torch.zeros(n_sample, self.params.d, dtype=torch.float32, device=_DEVICE) + epsilon

    def transform_grid(self, grid, theta):
        """Integrate ``grid`` ([ndim, nP] or [n_batch, ndim, nP]) under each theta.

        Output: [n_batch, ndim, nP].
        """
        if len(grid.shape) == 3:
            assert grid.shape[0] == theta.shape[0], \
                'When passing a batched grid, the first dimension must match theta'
        return transformer(grid, theta, self.params, compute_points_grad=True)

    def transform_grid_chain(self, grid, theta_chain, scale_by_dt=False):
        """Apply a time-ordered chain of CPAB transforms to a grid.

        Arguments:
            grid: [ndim, n_points] or [n_batch, ndim, n_points]
            theta_chain: [n_transforms, d] or [n_transforms, n_batch, d]
            scale_by_dt: bool, scale each stage by dt = 1 / n_transforms
        Output:
            [n_batch, ndim, n_points]
        """
        assert type(scale_by_dt) == bool, 'scale_by_dt must be bool'
        assert theta_chain.dim() in (2, 3), \
            'theta_chain must have shape [n_transforms, d] or [n_transforms, n_batch, d]'
        if theta_chain.dim() == 2:
            theta_chain = theta_chain[:, None, :]
        n_transforms, n_batch, d = theta_chain.shape
        assert n_transforms > 0, 'theta_chain must contain at least one transform'
        assert d == self.params.d, f'theta_chain has d={d}, expected d={self.params.d}'
        if grid.dim() == 3:
            assert grid.shape[0] == n_batch, \
                'When passing a 3D grid, its batch dimension must match theta_chain'
        dt = (1.0 / n_transforms) if scale_by_dt else 1.0
        # One forward and one backward launch for all stages; stage i uses
        # theta_chain[i] * dt exactly as the reference's per-stage loop does.
        return chain_transformer(grid, theta_chain * dt, self.params)

    def interpolate(self, data, grid, outsize):
        """Border-clamped linear interpolation of ``data`` at ``grid``; its data
        gradient is deterministic under ``set_solver_params(deterministic_grad=True)``."""
        return interpolate(self.params.ndim, data, grid, outsize,
                           deterministic=bool(getattr(self.params, "deterministic_grad", False)))

    def transform_data(self, data, theta, outsize):
        """Warp ``data`` [n_batch, C, *in_size] by theta onto an ``outsize`` grid.

        Same result as ``interpolate(data, transform_grid(uniform_meshgrid(outsize),
        theta), outsize)`` (cpab/cpab.py:295-309), computed by one fused
        forward and one fused backward launch: the warped grid never goes
        through HBM.
        """
        return transform_data_fused(data, theta, self._uniform_axes(outsize), outsize,
                                    self.params)

    def _uniform_axes(self, outsize):
        # The per-axis coordinates uniform_meshgrid takes the Cartesian product
        # of, concatenated; deterministic, so one per output size is kept
        # (internal use only, never handed to callers).
        key = tuple(int(v) for v in outsize)
        cache = self.__dict__.setdefault("_uniform_axes_cache", {})
        if key not in cache:
            cache[key] = torch.cat(self._linspaces(list(key)))
        return cache[key]

    def _linspaces(self, n_points):
        return [torch.linspace(self.params.domain_min[i], self.params.domain_max[i],
                               n_points[i], device=_DEVICE) for i in range(self.params.ndim)]

    def _check_input(self, tess_size, zero_boundary, volume_perservation, override):
        assert type(tess_size) in [list, tuple], 'tess_size must be a list or tuple'
        assert len(tess_size) in [1, 2, 3], 'Only 1D, 2D, and 3D tesselations are supported'
        assert all([type(e) == int for e in tess_size]), 'All elements must be integers'
        assert all([e > 0 for e in tess_size]), 'All elements must be positive'
        assert type(zero_boundary) == bool, 'zero_boundary must be True or False'
        assert type(volume_perservation) == bool, 'volume_perservation must be True or False'
        assert type(override) == bool, 'override must be True or False'

    def __repr__(self):
        return f'''
        CPAB transformer class ({self.params.ndim}D PyTorch HIP / MI355X).
            Parameters:
                Tesselation size:           {self.params.nc}
                Total number of cells:      {self.params.nC}
                Theta size:                 {self.params.d}
                Domain lower bound:         {self.params.domain_min}
                Domain upper bound:         {self.params.domain_max}
                Zero Boundary:              {self.params.zero_boundary}
                Volume perservation:        {self.params.volume_perservation}
        '''
