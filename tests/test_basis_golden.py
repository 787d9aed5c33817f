"""Basis parity against fixtures written by the reference's own tessellation
code (tests/golden/make_basis_fixtures.py, run once in the build container).

These pin what the closed forms in test_basis.py leave open: the SVD
null-space basis for zero_boundary=False / volume_perservation=True
(utility.py:36-56, tesselation.py:282-290), whose columns are fixed only up
to rotation by the mathematics, and the 1D/3D nodal column order
(tesselation.py:216-307).  With the same numpy/scipy as this image the
basis must agree exactly; the cell vertices (find_verts) too."""
import shutil

import numpy as np
import pytest
import scipy.sparse as sp

from cpab.core.tesselation import Tesselation1D, Tesselation2D, Tesselation3D

from golden.make_basis_fixtures import CASES, PICKLE_CASES, cache_name, fixture_name
from conftest import GOLDEN


def _load(nc, zb, vp):
    f = np.load(GOLDEN / fixture_name(nc, zb, vp))
    B = sp.csr_matrix((f["data"], f["indices"], f["indptr"]), shape=tuple(f["shape"]))
    return B.toarray(), f["verts"]


@pytest.mark.parametrize("nc,zb,vp", CASES)
def test_basis_matches_reference_fixture(nc, zb, vp):
    B_ref, verts_ref = _load(nc, zb, vp)
    n = len(nc)
    T = {1: Tesselation1D, 2: Tesselation2D, 3: Tesselation3D}[n](nc, [0] * n, [1] * n, zb, vp, None)
    np.testing.assert_array_equal(np.asarray(T.verts), verts_ref)
    B = T.B.toarray()
    assert B.shape == B_ref.shape
    np.testing.assert_allclose(B, B_ref, rtol=0, atol=1e-12)
    if B.size:
        # the subspace (what the velocity fields span), independent of the exact columns
        np.testing.assert_allclose(B @ B.T, B_ref @ B_ref.T, rtol=0, atol=1e-10)


@pytest.mark.parametrize("nc,zb,vp", PICKLE_CASES)
def test_reads_reference_written_cache(tmp_path, nc, zb, vp):
    # A basis_files/ cache written by the reference's own save_obj
    # (tesselation.py:101-104, utility.py:70-73) is read back through this
    # package's restricted loader, under the reference's file name, and holds
    # the same basis this package computes.
    name = cache_name(nc, zb, vp)
    shutil.copy(GOLDEN / ("refcache_" + name + ".pkl"), tmp_path / (name + ".pkl"))
    n = len(nc)
    cls = {1: Tesselation1D, 2: Tesselation2D, 3: Tesselation3D}[n]
    T = cls(nc, [0] * n, [1] * n, zb, vp, str(tmp_path) + "/")
    # loaded, not recomputed: the dict carries the folder the reference wrote it to
    assert T.dir != str(tmp_path) + "/"
    assert T._basis_file.endswith(name)
    fresh = cls(nc, [0] * n, [1] * n, zb, vp, None)
    assert sp.issparse(T.B) and T.B.shape == fresh.B.shape
    np.testing.assert_allclose(T.B.toarray(), fresh.B.toarray(), rtol=0, atol=1e-12)
    np.testing.assert_array_equal(np.asarray(T.verts), np.asarray(fresh.verts))
    assert int(T.nC) == int(fresh.nC)
