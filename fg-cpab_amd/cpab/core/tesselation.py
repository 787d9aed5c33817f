"""Tessellations of [0,1]^n and the CPA velocity basis ``B``.

Host-side set-up (CPU, float64, run once per tessellation and cached under
``basis_files/``).  The public surface follows the reference's
``cpab/core/tesselation.py``: classes ``Tesselation1D/2D/3D`` with the
constructor ``(nc, domain_min, domain_max, zero_boundary, volume_perservation,
direc, override)`` and the attributes ``verts, cells, L, B, nC, ndim,
n_params, nodal_vertices, shared_v, shared_v_idx``.

Three things here are interfaces and therefore kept identical to the
reference, in code of our own:

* the cell / vertex enumeration ("order matters"), because the HIP cell lookup
  and the theta coordinates depend on it (``tesselation.py:322-335,362-390,
  470-513``);
* the nodal basis: ``B = N`` column-normalised, where ``N`` maps the velocity
  of every active (non-boundary if ``zero_boundary``) vertex, in first-seen
  order over the cells, onto the per-cell affine parameters
  (``tesselation.py:216-307``).  When every residual constraint ``L N`` is
  numerically zero (the case for ``zero_boundary=True`` without volume
  preservation) this is the whole basis; otherwise the residual constraints are
  projected out with an SVD null space (``utility.py:36-56``), which is unique
  only up to a rotation of the null space;
* the cache file name ``cpab_basis_dim{n}_tess{a_b}_vo{}_zb{}_vp{}_nodal_v2.pkl``
  and its ``__dict__`` payload (``tesselation.py:64-71,101,104``).
"""
from itertools import combinations

import numpy as np
import scipy.sparse as sp

from .utility import (check_if_file_exist, drop_zero_rows, load_obj,
                      make_hashable, null, save_obj)

_BASIS_VERSION = "nodal_v2"


class Tesselation(object):
    """Shared machinery; subclasses supply the cell geometry."""

    def __init__(self, nc, domain_min, domain_max, zero_boundary=True,
                 volume_perservation=False, direc=None, override=False):
        self.nc = nc
        self.domain_min = domain_min
        self.domain_max = domain_max
        self.zero_boundary = zero_boundary
        self.volume_perservation = volume_perservation
        self.dir = direc
        self._basis_file = (
            (direc or "") + "cpab_basis_dim" + str(len(nc)) + "_tess"
            + "_".join(str(e) for e in nc)
            + "_vo" + str(int(not zero_boundary))
            + "_zb" + str(int(zero_boundary))
            + "_vp" + str(int(volume_perservation))
            + "_" + _BASIS_VERSION)

        if override or direc is None or not check_if_file_exist(self._basis_file + ".pkl"):
            self._build()
            if direc is not None:
                save_obj(self.__dict__, self._basis_file)
        else:
            self.__dict__ = load_obj(self._basis_file)
            if not sp.issparse(self.L):
                self.L = sp.csr_matrix(self.L)
            if not sp.issparse(self.B):
                self.B = sp.csr_matrix(self.B)

    # -- construction -------------------------------------------------------
    def _build(self):
        self.find_verts()
        self.find_shared_verts()
        if not self.zero_boundary:
            self.find_verts_outside()
        blocks = [self.create_continuity_constrains()]
        if self.zero_boundary:
            blocks.append(self.create_zero_boundary_constrains())
        if self.volume_perservation:
            blocks.append(self.create_zero_trace_constrains())
        self.L = sp.vstack(blocks, format="csr") if len(blocks) > 1 else blocks[0].tocsr()
        self.B = self.create_nodal_basis_sparse()

    def get_cell_centers(self):
        """Mean of each cell's vertices, ``[nC, ndim]``."""
        return np.mean(self.verts[:, :, :self.ndim], axis=1)

    def find_verts(self):
        raise NotImplementedError

    def find_verts_outside(self):
        raise NotImplementedError

    def create_zero_boundary_constrains(self):
        raise NotImplementedError

    def find_shared_verts(self):
        """Pairs of cells sharing an (ndim-1)-face, in first-seen face order.

        A face is any ``ndim`` of a cell's ``ndim+1`` vertices, keyed by its
        sorted vertex tuples; every pair of cells listing the same face gets a
        continuity constraint (``tesselation.py:119-146``).
        """
        owners = {}
        for c in range(self.nC):
            for face in combinations(make_hashable(self.verts[c]), self.ndim):
                owners.setdefault(tuple(sorted(face)), []).append(c)
        faces, pairs = [], []
        for face, cells in owners.items():
            for a in range(len(cells)):
                for b in range(a + 1, len(cells)):
                    faces.append(list(face))
                    pairs.append((cells[a], cells[b]))
        self.shared_v = (np.asarray(faces) if faces
                         else np.zeros((0, self.ndim, self.ndim)))
        self.shared_v_idx = pairs

    def create_continuity_constrains(self):
        """Rows ``v . (A_i[k,:] - A_j[k,:]) = 0`` for each shared vertex ``v``
        of each shared face and each output dimension ``k``."""
        nd, npar = self.ndim, self.n_params
        rows, cols, vals = [], [], []
        r = 0
        for idx, (ci, cj) in enumerate(self.shared_v_idx):
            for vidx in range(nd):
                v = np.asarray(self.shared_v[idx][vidx], dtype=np.float64)
                nz = np.flatnonzero(v != 0.0)
                for k in range(nd):
                    off_i = npar * ci + k * (nd + 1)
                    off_j = npar * cj + k * (nd + 1)
                    for q in nz:
                        rows += [r, r]
                        cols += [off_i + q, off_j + q]
                        vals += [v[q], -v[q]]
                    r += 1
        n_rows = len(self.shared_v_idx) * nd * nd
        return sp.coo_matrix((vals, (rows, cols)),
                             shape=(n_rows, npar * self.nC)).tocsr()

    def _boundary_rows(self):
        """Zero normal velocity at boundary vertices: a vertex on the x-min/max
        face constrains row 0 of the cell's affine map, y row 1, z row 2
        (``tesselation.py:431-455,547-578``)."""
        nd, npar = self.ndim, self.n_params
        rows, cols, vals = [], [], []
        r = 0
        for c in range(self.nC):
            for v in self.verts[c]:
                for k in range(nd):
                    if v[k] == self.domain_min[k] or v[k] == self.domain_max[k]:
                        for q, value in enumerate(v):
                            if value != 0.0:
                                rows.append(r)
                                cols.append(npar * c + k * (nd + 1) + q)
                                vals.append(value)
                        r += 1
        return sp.coo_matrix((vals, (rows, cols)), shape=(r, npar * self.nC)).tocsr()

    def create_zero_trace_constrains(self):
        """One row per cell: trace of the linear part is zero."""
        nd, npar = self.ndim, self.n_params
        rows = np.repeat(np.arange(self.nC), nd)
        cols = (npar * np.arange(self.nC)[:, None]
                + np.arange(nd)[None, :] * (nd + 2)).ravel()
        vals = np.ones(rows.size)
        return sp.coo_matrix((vals, (rows, cols)),
                             shape=(self.nC, npar * self.nC)).tocsr()

    def _is_boundary_vertex(self, vertex, atol=1e-12):
        return any(np.isclose(vertex[k], self.domain_min[k], atol=atol)
                   or np.isclose(vertex[k], self.domain_max[k], atol=atol)
                   for k in range(self.ndim))

    def create_nodal_prolongation(self):
        """Sparse ``N [D, ndim * n_active]``: nodal velocities -> affine params.

        For cell ``c`` with homogeneous vertices as rows of ``V_c``, the affine
        map interpolating vertex velocities ``U`` (columns) is ``U V_c^{-T}``,
        so vertex ``l``'s velocity component ``k`` enters ``A_c[k, q]`` with
        weight ``(V_c^{-T})[l, q]``.  Column ``ndim * a + k`` belongs to active
        vertex ``a`` (first-seen order), component ``k``.
        """
        nd, npar = self.ndim, self.n_params
        order = {}
        for c in range(self.nC):
            for v in self.verts[c]:
                order.setdefault(tuple(np.asarray(v, dtype=np.float64).tolist()), None)
        active = {}
        for key in order:
            if self.zero_boundary and self._is_boundary_vertex(key):
                continue
            active[key] = len(active)
        self.nodal_vertices = np.asarray(list(active.keys()))
        D = npar * self.nC
        if not active:
            return sp.csr_matrix((D, 0))
        V = np.asarray(self.verts, dtype=np.float64)
        Vinv = np.stack([np.linalg.inv(V[c].T) for c in range(self.nC)])
        rows, cols, vals = [], [], []
        for c in range(self.nC):
            for l, v in enumerate(V[c]):
                a = active.get(tuple(v.tolist()))
                if a is None:
                    continue
                coeff = Vinv[c, l]
                nz = np.flatnonzero(coeff != 0.0)
                for k in range(nd):
                    base = npar * c + k * (nd + 1)
                    rows.extend((base + nz).tolist())
                    cols.extend([nd * a + k] * nz.size)
                    vals.extend(coeff[nz].tolist())
        N = sp.coo_matrix((vals, (rows, cols)), shape=(D, nd * len(active))).tocsr()
        N.eliminate_zeros()
        return N

    def create_nodal_basis_sparse(self, eps=1e-6):
        N = self.create_nodal_prolongation()
        C = (self.L @ N).tocsr()
        if C.nnz:
            C.data[np.abs(C.data) <= eps] = 0.0
            C.eliminate_zeros()
        C = drop_zero_rows(C)
        if C.shape[0] == 0 or C.shape[1] == 0:
            return self._normalize_basis_columns(N)
        Z = null(C, eps=eps, zero_tol=eps)
        if Z.shape[1] == 0:
            return sp.csr_matrix((N.shape[0], 0))
        B = (N @ Z).tocsr()
        if B.nnz:
            B.data[np.abs(B.data) <= eps] = 0.0
            B.eliminate_zeros()
        return self._normalize_basis_columns(B)

    @staticmethod
    def _normalize_basis_columns(B):
        if B.shape[1] == 0:
            return B.tocsr()
        Bc = B.tocsc(copy=True)
        norms = np.sqrt(np.asarray(Bc.power(2).sum(axis=0)).ravel())
        norms[norms == 0.0] = 1.0
        counts = np.diff(Bc.indptr)
        Bc.data /= np.repeat(norms, counts)
        Bc.eliminate_zeros()
        return Bc.tocsr()


class Tesselation1D(Tesselation):
    """``nc[0]`` intervals; cell ``i`` spans ``[x_i, x_{i+1}]``."""

    def __init__(self, nc, domain_min, domain_max, zero_boundary=True,
                 volume_perservation=False, direc=None, override=False):
        self.n_params = 2
        self.nC = int(np.prod(nc))
        self.ndim = 1
        super().__init__(nc, domain_min, domain_max, zero_boundary,
                         volume_perservation, direc, override)

    def find_verts(self):
        Vx = np.linspace(self.domain_min[0], self.domain_max[0], self.nc[0] + 1)
        self.verts = np.stack([np.stack([Vx[:-1], np.ones(self.nc[0])], 1),
                               np.stack([Vx[1:], np.ones(self.nc[0])], 1)], 1)
        self.cells = list(range(self.nc[0]))

    def find_verts_outside(self):
        pass  # a 1D field extends past the ends without extra constraints

    def create_zero_boundary_constrains(self):
        n = 2 * self.nC
        return sp.coo_matrix(([self.domain_min[0], 1.0, self.domain_max[0], 1.0],
                              ([0, 0, 1, 1], [0, 1, n - 2, n - 1])),
                             shape=(2, n)).tocsr()


class Tesselation2D(Tesselation):
    """``nc[0] x nc[1]`` squares, each cut into 4 triangles around its centre.

    Cell ``4 * (jx + iy * nc[0]) + t`` with ``t`` = 0 top (y-min edge),
    1 right, 2 bottom, 3 left; each triangle lists the centre first.
    """

    def __init__(self, nc, domain_min, domain_max, zero_boundary=True,
                 volume_perservation=False, direc=None, override=False):
        self.n_params = 6
        self.nC = 4 * int(np.prod(nc))
        self.ndim = 2
        super().__init__(nc, domain_min, domain_max, zero_boundary,
                         volume_perservation, direc, override)

    def find_verts(self):
        Vx = np.linspace(self.domain_min[0], self.domain_max[0], self.nc[0] + 1)
        Vy = np.linspace(self.domain_min[1], self.domain_max[1], self.nc[1] + 1)
        verts, cells = [], []
        for iy in range(self.nc[1]):
            for jx in range(self.nc[0]):
                x0, x1, y0, y1 = Vx[jx], Vx[jx + 1], Vy[iy], Vy[iy + 1]
                ce = ((x0 + x1) / 2, (y0 + y1) / 2, 1)
                ul, ur, ll, lr = (x0, y0, 1), (x1, y0, 1), (x0, y1, 1), (x1, y1, 1)
                verts += [(ce, ul, ur), (ce, ur, lr), (ce, lr, ll), (ce, ll, ul)]
                cells += [(jx, iy, t) for t in range(4)]
        self.verts = np.asarray(verts)
        self.cells = cells

    def find_verts_outside(self):
        """Continuity of the extension past the domain: boundary triangles of
        neighbouring squares that meet in one boundary vertex get a constraint
        at that vertex and at an auxiliary point 10 units away
        (``tesselation.py:392-429``)."""
        nx, ny = self.nc[0], self.nc[1]
        index = {tuple(self.cells[k]): k for k in range(self.nC)}
        faces, pairs = [], []
        for i in range(self.nC):
            jx, iy, t = self.cells[i]
            side_x = (jx == 0 and t == 3) or (jx == nx - 1 and t == 1)
            side_y = (iy == 0 and t == 0) or (iy == ny - 1 and t == 2)
            cand = []
            if jx == 0 and t == 3:
                cand += [(0, iy + 1, 3), (0, iy - 1, 3)]
            if jx == nx - 1 and t == 1:
                cand += [(nx - 1, iy + 1, 1), (nx - 1, iy - 1, 1)]
            if iy == 0 and t == 0:
                cand += [(jx + 1, 0, 0), (jx - 1, 0, 0)]
            if iy == ny - 1 and t == 2:
                cand += [(jx + 1, ny - 1, 2), (jx - 1, ny - 1, 2)]
            for key in cand:
                j = index.get(key)
                if j is None or not i < j:
                    continue
                common = set(make_hashable(self.verts[i])).intersection(
                    make_hashable(self.verts[j]))
                if len(common) != 1:
                    continue
                shared = tuple(common)[0]
                aux = list(shared)
                if side_x:
                    aux[0] -= 10
                elif side_y:
                    aux[1] -= 10
                faces.append([shared, tuple(aux)])
                pairs.append((i, j))
        if faces:
            self.shared_v = np.concatenate((self.shared_v, faces))
            self.shared_v_idx += pairs

    def create_zero_boundary_constrains(self):
        return self._boundary_rows()


class Tesselation3D(Tesselation):
    """``nc[0] x nc[1] x nc[2]`` cubes, each cut into 5 tetrahedra (one
    central); odd-parity cubes use the mirrored cut so faces match."""

    def __init__(self, nc, domain_min, domain_max, zero_boundary=True,
                 volume_perservation=False, direc=None, override=False):
        self.n_params = 12
        self.nC = 5 * int(np.prod(nc))
        self.ndim = 3
        super().__init__(nc, domain_min, domain_max, zero_boundary,
                         volume_perservation, direc, override)

    def find_verts(self):
        Vx = np.linspace(self.domain_min[0], self.domain_max[0], self.nc[0] + 1)
        Vy = np.linspace(self.domain_min[1], self.domain_max[1], self.nc[1] + 1)
        Vz = np.linspace(self.domain_min[2], self.domain_max[2], self.nc[2] + 1)
        verts, cells = [], []
        for iz in range(self.nc[2]):
            for jy in range(self.nc[1]):
                for kx in range(self.nc[0]):
                    def corner(dx, dy, dz):
                        return (Vx[kx + dx], Vy[jy + dy], Vz[iz + dz], 1)
                    q0 = [corner(0, 0, 0), corner(1, 0, 0), corner(1, 1, 0), corner(0, 1, 0)]
                    q1 = [corner(0, 0, 1), corner(1, 0, 1), corner(1, 1, 1), corner(0, 1, 1)]
                    if (iz + jy + kx) % 2 == 1:  # rotate the cut by one corner
                        q0 = q0[1:] + q0[:1]
                        q1 = q1[1:] + q1[:1]
                    ul0, ur0, lr0, ll0 = q0
                    ul1, ur1, lr1, ll1 = q1
                    verts += [(ll1, ur1, ul0, lr0), (ul1, ur1, ll1, ul0),
                              (lr1, ur1, ll1, lr0), (ll0, ul0, lr0, ll1),
                              (ur0, ul0, lr0, ur1)]
                    cells += [(kx, jy, iz, t) for t in range(5)]
        self.verts = np.asarray(verts)
        self.cells = cells

    def find_verts_outside(self):
        """Two tetrahedra of one cube that both own a face on the same domain
        face share a constraint at their common edge plus an auxiliary point
        one unit outside (``tesselation.py:515-544``)."""
        faces, pairs = [], []
        for cube in range(self.nC // 5):
            for a in range(5):
                for b in range(a + 1, 5):
                    i, j = 5 * cube + a, 5 * cube + b
                    vi, vj = self.verts[i], self.verts[j]
                    for k in range(self.ndim):
                        on_min = (np.sum(vi[:, k] == self.domain_min[k]) == 3
                                  and np.sum(vj[:, k] == self.domain_min[k]) == 3)
                        on_max = (np.sum(vi[:, k] == self.domain_max[k]) == 3
                                  and np.sum(vj[:, k] == self.domain_max[k]) == 3)
                        if not (on_min or on_max):
                            continue
                        hi, hj = make_hashable(vi), make_hashable(vj)
                        common = set(hi).intersection(hj)
                        mid = [(p + q) / 2.0 for p, q in zip(hi[0], hj[0])]
                        mid[k] += -1 if on_min else 1
                        faces.append(list(common.union([tuple(mid)])))
                        pairs.append((i, j))
        if faces:
            self.shared_v = np.concatenate((self.shared_v, np.asarray(faces)))
            self.shared_v_idx += pairs

    def create_zero_boundary_constrains(self):
        return self._boundary_rows()
