"""Small host-side helpers shared by the tessellation and the Cpab API.

Mirrors the helper surface of the reference's ``cpab/core/utility.py``
(``params`` container, directory helpers, null space, pickle cache I/O), with
one deliberate difference: cached basis files are read back through a
restricted unpickler that resolves only an exact list of globals (numpy's
array, scalar and dtype reconstructors, scipy.sparse's csr / csc / coo classes
and builtin containers), so a cache file cannot name any callable that runs
code or touches files.
"""
import os
import pickle
import io

import numpy as np
import scipy.linalg as la
import scipy.sparse as sp


class params:
    """Attribute bag holding the transformation parameters.

    Same role and field names as ``params`` in the reference
    (``cpab/core/utility.py:11-16``; fields filled at ``cpab/cpab.py:31-43,73-79``).
    """

    def __repr__(self):
        return str(self.__dict__)


def get_dir(file):
    """Directory holding ``file`` (symlinks resolved)."""
    return os.path.dirname(os.path.realpath(file))


def create_dir(direc):
    """Create ``direc`` if it is missing (tolerates concurrent creation)."""
    os.makedirs(direc, exist_ok=True)


def check_if_file_exist(file):
    return os.path.isfile(file)


def make_hashable(arr):
    """Rows of a 2-D array as a tuple of tuples (usable as dict keys)."""
    return tuple(tuple(r.tolist()) for r in np.asarray(arr))


def drop_zero_rows(A):
    """Remove rows without stored non-zeros (sparse) or all-zero rows (dense).

    Same contract as ``drop_zero_rows`` at ``cpab/core/utility.py:19-33``.
    """
    if sp.issparse(A):
        A = A.tocsr()
        keep = np.flatnonzero(np.diff(A.indptr))
        return A if keep.size == A.shape[0] else A[keep]
    A = np.asarray(A)
    if A.ndim != 2:
        raise ValueError("Expected a 2D matrix")
    return A[np.flatnonzero(np.any(np.abs(A) > 0, axis=1))]


def null(A, eps=1e-6, zero_tol=None):
    """Null space of ``A`` as a sparse CSR matrix with one basis vector per column.

    Follows ``cpab/core/utility.py:36-56``: full SVD, singular values ``<= eps``
    (plus the rank-deficient tail) select rows of ``V^H``; entries with
    magnitude ``<= zero_tol`` (default ``eps``) are zeroed.  The basis returned
    by an SVD is unique only up to a rotation of the null space, so the exact
    columns depend on the LAPACK build.
    """
    if sp.issparse(A):
        A = A.toarray()
    A = np.asarray(A, dtype=np.float64)
    if A.ndim != 2:
        raise ValueError("Expected a 2D matrix")
    if A.shape[1] == 0:
        return sp.csr_matrix((0, 0))
    _, s, vh = la.svd(A)
    tail = max(0, A.shape[1] - s.shape[0])
    mask = np.concatenate((s <= eps, np.ones(tail, dtype=bool)))
    Z = vh[mask].T.copy()
    Z[np.abs(Z) <= (eps if zero_tol is None else zero_tol)] = 0.0
    Z = sp.csr_matrix(Z)
    Z.eliminate_zeros()
    return Z


# ---------------------------------------------------------------------------
# Basis cache I/O
# ---------------------------------------------------------------------------

# The exact globals a cached tessellation dict may reference, as the
# reference's save_obj (pickle.dump of Tesselation.__dict__, utility.py:70-73,
# tesselation.py:101) writes them under numpy 1.x / 2.x and scipy's old and
# new module layouts: array and scalar reconstructors, dtype, and the sparse
# matrix classes (rebuilt from their state, without calling __init__).  Every
# other global, in numpy or anywhere else, is refused.
_NUMPY_CORE = ("numpy.core", "numpy._core")
_SAFE_GLOBALS = frozenset(
    [("numpy", "dtype"), ("numpy", "ndarray")]
    + [(c + ".multiarray", n) for c in _NUMPY_CORE for n in ("_reconstruct", "scalar")]
    + [(c + ".numeric", "_frombuffer") for c in _NUMPY_CORE]
    + [(m, k + "_" + kind)
       for k in ("csr", "csc", "coo")
       for m in ("scipy.sparse", "scipy.sparse." + k, "scipy.sparse._" + k)
       for kind in ("matrix", "array")]
    + [("builtins", n) for n in ("dict", "list", "tuple", "set", "frozenset", "int", "float",
                                  "complex", "bool", "str", "bytes", "bytearray", "slice", "range")])


class _RestrictedUnpickler(pickle.Unpickler):
    def find_class(self, module, name):
        if (module, name) in _SAFE_GLOBALS:
            return super().find_class(module, name)
        raise pickle.UnpicklingError(f"refusing to load global {module}.{name}")


def load_obj(name):
    """Load ``name + '.pkl'`` through the restricted unpickler."""
    with open(name + ".pkl", "rb") as f:
        return _RestrictedUnpickler(io.BytesIO(f.read())).load()


def save_obj(obj, name):
    """Write ``obj`` to ``name + '.pkl'`` atomically (temp file + rename)."""
    tmp = f"{name}.pkl.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        pickle.dump(obj, f, pickle.HIGHEST_PROTOCOL)
    os.replace(tmp, name + ".pkl")
