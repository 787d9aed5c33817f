"""Writes tests/golden/basis_*.npz from the reference's own tessellation code.

Runs in the build container only (it needs the reference checkout at
/root/reference; nothing at test time reads the reference).  The reference's
cpab/core/{utility,tesselation}.py are loaded by file path under a private
package name, so cpab/__init__.py (which JIT-builds the CUDA extension) is not
executed; the basis cache the reference writes goes to a temporary folder.

Fixtures pin what no closed form here fixes: the SVD null-space basis for
zero_boundary=False / volume_perservation=True (utility.py:36-56,
tesselation.py:282-290) and the 1D/3D nodal-basis column order
(tesselation.py:216-307).  Each .npz holds the CSR arrays of B, its shape and
the cell vertices (verts) of the tessellation.

It also keeps, for PICKLE_CASES, the basis cache file exactly as the
reference's Tesselation writes it through its save_obj (pickle of the
instance __dict__, tesselation.py:101-104, utility.py:70-73), as
refcache_<cache file name>.pkl: data for the test that this package's
restricted loader reads caches the reference left in a basis_files/ folder.
"""
import importlib.util
import os
import sys
import tempfile
import types

import numpy as np
import scipy.sparse as sp

REF = os.environ.get("CPAB_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.realpath(__file__))

CASES = [
    # (nc, zero_boundary, volume_perservation)
    ([5], False, False),
    ([5], True, True),
    ([6], True, False),
    ([4, 3], False, False),
    ([4, 3], True, True),
    ([3, 4], True, False),
    ([2, 2, 2], False, False),
    ([2, 2, 2], False, True),
    ([2, 3, 2], True, False),
    ([3, 3, 3], True, False),
]


def load_reference_core():
    pkg = types.ModuleType("_refcore")
    pkg.__path__ = [os.path.join(REF, "cpab", "core")]
    sys.modules["_refcore"] = pkg
    mods = {}
    for name in ("utility", "tesselation"):
        spec = importlib.util.spec_from_file_location(
            "_refcore." + name, os.path.join(REF, "cpab", "core", name + ".py"))
        m = importlib.util.module_from_spec(spec)
        sys.modules["_refcore." + name] = m
        spec.loader.exec_module(m)
        mods[name] = m
    return mods["tesselation"]


# Small cases whose reference-written cache file is kept (1D through the SVD
# null space, 2D through the nodal basis).
PICKLE_CASES = [
    ([5], False, False),
    ([3, 2], True, False),
]


def cache_name(nc, zb, vp):
    """The reference's cache file name (tesselation.py:64-71), without .pkl."""
    return ("cpab_basis_dim%d_tess%s_vo%d_zb%d_vp%d_nodal_v2"
            % (len(nc), "_".join(map(str, nc)), int(not zb), int(zb), int(vp)))


def fixture_name(nc, zb, vp):
    return "basis_%s_zb%d_vp%d.npz" % ("x".join(map(str, nc)), int(zb), int(vp))


def main():
    tess = load_reference_core()
    cls = {1: tess.Tesselation1D, 2: tess.Tesselation2D, 3: tess.Tesselation3D}
    with tempfile.TemporaryDirectory() as tmp:
        for nc, zb, vp in CASES:
            n = len(nc)
            T = cls[n](nc, [0] * n, [1] * n, zb, vp, tmp + "/", True)
            B = sp.csr_matrix(T.B)
            np.savez_compressed(os.path.join(HERE, fixture_name(nc, zb, vp)),
                                data=B.data, indices=B.indices, indptr=B.indptr,
                                shape=np.array(B.shape), verts=np.asarray(T.verts, dtype=np.float64))
            print(fixture_name(nc, zb, vp), B.shape, B.nnz)
        for nc, zb, vp in PICKLE_CASES:
            n = len(nc)
            # override=True: computed and saved by the reference's own save_obj
            cls[n](nc, [0] * n, [1] * n, zb, vp, tmp + "/", True)
            src = os.path.join(tmp, cache_name(nc, zb, vp) + ".pkl")
            with open(src, "rb") as f_in, open(os.path.join(HERE, "refcache_" + cache_name(nc, zb, vp) + ".pkl"), "wb") as f_out:
                f_out.write(f_in.read())
            print("refcache_" + cache_name(nc, zb, vp) + ".pkl")


if __name__ == "__main__":
    main()
