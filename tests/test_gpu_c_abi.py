"""libcpab_hip.so called from plain C (tests/c_abi/cpab_c_caller.c, built by
__graft_entry__.build()): the calls a C / C++ / cgo / JNI host makes, with its
own device memory and stream from the HIP runtime's C API and no torch on the
path.  The C code runs in this process, loaded as a shared library (a GPU
process here starts no other program).  The forward points match the oracle
bit for bit; the moments and point adjoints within the GPU tests'
tolerances."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as orc

from helpers import assert_adjoint_close, assert_grad_close

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.realpath(__file__)), "c_abi", "libcpab_c_caller.so")
# the caller's problem (cpab_c_caller.c): 2D [4, 4], identity basis, 2 thetas,
# 1000 shared points, 50 steps
NC, NTHETA, NP, T = 64, 2, 1000, 50


def test_c_caller_matches_oracle(cuda, tmp_path):
    if not os.path.isfile(LIB):
        pytest.fail(f"{LIB} is missing: build it with __graft_entry__.build() "
                    "(make -C tests/c_abi)")
    caller = ctypes.CDLL(LIB)
    caller.cpab_c_caller_run.argtypes = [ctypes.c_char_p]
    caller.cpab_c_caller_run.restype = ctypes.c_int
    out = tmp_path / "c_caller.bin"
    assert caller.cpab_c_caller_run(str(out).encode()) == 0
    a = np.fromfile(out, dtype=np.float32)
    sizes = [NTHETA * NC * 6, 2 * NP, NTHETA * 2 * NP, NTHETA * 2 * NP, NTHETA * NC * 6,
             NTHETA * 2 * NP]
    assert a.size == sum(sizes)
    theta, pts, gout, got_out, got_m, got_gp = np.split(a, np.cumsum(sizes)[:-1])
    As = theta.reshape(NTHETA, NC, 2, 3)   # identity basis: A = theta
    pts = pts.reshape(2, NP)
    gout = gout.reshape(NTHETA, 2, NP)
    ref_out = orc.forward_trels(pts, orc.expm(2, As, 1.0 / T), As, [4, 4], T)
    np.testing.assert_array_equal(got_out.reshape(NTHETA, 2, NP), ref_out)
    ref_m, ref_gp = orc.backward(pts, As, gout, [4, 4], T)
    assert_grad_close(got_m.reshape(NTHETA, -1), ref_m.reshape(NTHETA, -1))
    assert_adjoint_close(got_gp.reshape(NTHETA, 2, NP), ref_gp)
