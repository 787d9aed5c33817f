"""C ABI checks that need no GPU: the library loads, exports every symbol
include/cpab_hip.h declares, and rejects bad arguments before any HIP call
(the reference's TORCH_CHECK set, transformer_cuda.cu:38-48,183-197).

The argument checks pass made-up device addresses that validation must
reject before anything is launched.  They run in a child process that sees
no GPU (HIP_VISIBLE_DEVICES=-1, ROCR_VISIBLE_DEVICES=-1, set before the
library initialises HIP), so that if validation ever let a call through, the
launch would fail with a HIP error instead of touching those addresses."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from cpab.pytorch import _native

ROOT = os.path.dirname(os.path.dirname(os.path.realpath(__file__)))
HERE = os.path.dirname(os.path.realpath(__file__))


def _run_without_gpu(check):
    """Run the module-level function `check` of this file in a child process
    with every GPU hidden."""
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1",
               CUDA_VISIBLE_DEVICES="-1")
    paths = [HERE, ROOT, os.path.join(ROOT, "fg-cpab_amd")]
    code = f"import sys; sys.path[:0] = {paths!r}; import test_capi; test_capi.{check}()"
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr


def _declared():
    txt = open(os.path.join(ROOT, "include", "cpab_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(cpab_\w+)\s*\(", txt)))


def test_header_symbols_exported():
    lib = ctypes.CDLL(_native.LIB_PATH)
    declared = _declared()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.exported_symbols())


def test_abi_version():
    # 300: backward launches form the moments and project them (fused tail)
    assert _native.load_library().cpab_abi_version() >= 300


def _err(lib):
    return lib.cpab_last_error_string().decode()


def test_forward_rejects_bad_steps_and_ndim():
    _run_without_gpu("_check_forward_rejects_bad_steps_and_ndim")


def _check_forward_rejects_bad_steps_and_ndim():
    lib = _native.load_library()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.cpab_forward(2, 10, 1, 0, 101, 4, 4, 1, 0, p, p, p, p, None)
    assert rc == 1 and "CPAB_MAX_STEPS=100" in _err(lib)
    rc = lib.cpab_forward(2, 10, 1, 0, 0, 4, 4, 1, 0, p, p, p, p, None)
    assert rc == 1 and "nstepsolver > 0" in _err(lib)
    rc = lib.cpab_forward(4, 10, 1, 0, 50, 4, 4, 1, 0, p, p, p, p, None)
    assert rc == 1 and "ndim" in _err(lib)
    rc = lib.cpab_forward(2, 10, 1, 0, 50, 4, 4, 1, 2, p, p, p, p, None)
    assert rc == 1 and "adaptive_substeps" in _err(lib)
    rc = lib.cpab_forward(2, 10, 1, 0, 50, 0, 4, 1, 0, p, p, p, p, None)
    assert rc == 1 and "tessellation" in _err(lib)
    # cell ids are 24-bit: 2D 2048 x 2048 squares (2^24 triangles) is one too many
    rc = lib.cpab_forward(2, 10, 1, 0, 50, 2048, 2048, 1, 0, p, p, p, p, None)
    assert rc == 1 and "2^24" in _err(lib)
    rc = lib.cpab_forward(3, 10, 1, 0, 50, 256, 256, 52, 0, p, p, p, p, None)
    assert rc == 1 and "2^24" in _err(lib)


def test_backward_rejects_null_and_small_workspace():
    _run_without_gpu("_check_backward_rejects_null_and_small_workspace")


def _check_backward_rejects_null_and_small_workspace():
    lib = _native.load_library()
    p = ctypes.c_void_p(16)
    rc = lib.cpab_backward(2, 10, 1, 0, 50, 4, 4, 1, 0, p, p, p, None, None, None, 0, None)
    assert rc == 1 and "moments" in _err(lib)
    rc = lib.cpab_backward(3, 10, 1, 0, 101, 2, 2, 2, 0, p, p, p, p, None, None, 0, None)
    assert rc == 1 and "CPAB_MAX_STEPS" in _err(lib)


def test_trace_and_interp_validation():
    _run_without_gpu("_check_trace_and_interp_validation")


def _check_trace_and_interp_validation():
    lib = _native.load_library()
    p = ctypes.c_void_p(16)
    rc = lib.cpab_trace_cells(1, 10, 1, 0, 50, 4, 1, 1, 0, p, p, p, p, None)
    assert rc == 1
    sizes = (ctypes.c_int64 * 3)(4, 4, 4)
    rc = lib.cpab_interp_forward(4, 1, 1, sizes, sizes, p, p, p, None)
    assert rc == 1 and "ndim" in _err(lib)
    bad = (ctypes.c_int64 * 2)(0, 4)
    rc = lib.cpab_interp_forward(2, 1, 1, bad, sizes, p, p, p, None)
    assert rc == 1
    # the gathers address one data channel with 32-bit byte offsets: at most 2^30 values
    big = (ctypes.c_int64 * 3)(1024, 1024, 1025)
    rc = lib.cpab_interp_forward(3, 1, 1, big, sizes, p, p, p, None)
    assert rc == 1 and "2^30" in _err(lib)
    rc = lib.cpab_interp_backward(3, 1, 1, big, sizes, p, p, p, p, None, None)
    assert rc == 1 and "2^30" in _err(lib)
    huge = (ctypes.c_int64 * 3)(1 << 30, 1 << 30, 1 << 30)   # products beyond int64 if unchecked
    rc = lib.cpab_interp_forward(3, 1, 1, sizes, huge, p, p, p, None)
    assert rc == 1
    rc = lib.cpab_transform_data_forward(3, 1, 1, big, sizes, 50, 2, 2, 2, 0, p, p, p, p, p, None,
                                         None, None)
    assert rc == 1 and "2^30" in _err(lib)
    # The fused image calls index output positions with 32-bit ints and walk
    # them in grid strides (two positions per lane in 2D): the output must
    # stay below (2^31 - 1) / 3 positions, the point limit of cpab_forward.
    small = (ctypes.c_int64 * 2)(8, 8)
    for out in ((1 << 16, (1 << 15) - 2), (715827883, 1), ((1 << 31) - 1, 1)):
        outs = (ctypes.c_int64 * 2)(*out)
        rc = lib.cpab_transform_data_forward(2, 1, 1, small, outs, 50, 2, 2, 1, 0, p, p, p, p, p,
                                             None, None, None)
        assert rc == 1 and "32-bit point index" in _err(lib), out
        rc = lib.cpab_transform_data_backward(2, 1, 1, small, outs, 50, 2, 2, 1, 0, p, p, None, p,
                                              p, p, 0, None, None, None, p, None, None, p, 1 << 30,
                                              None)
        assert rc == 1 and "32-bit point index" in _err(lib), out
    rc = lib.cpab_forward(2, 715827882, 1, 0, 50, 2, 2, 1, 0, p, p, p, p, None)
    assert rc == 1 and "32-bit point index" in _err(lib)


def test_transform_data_seed_grad_checks():
    # seed_grad only with one channel; the backward needs final_points unless
    # seed_grad is given and grad_data is not.  Validation fails before any
    # launch (the pointers are never dereferenced).
    lib = _native.load_library()
    p = ctypes.c_void_p(64)
    ins = (ctypes.c_int64 * 2)(8, 8)
    outs = (ctypes.c_int64 * 2)(8, 8)
    rc = lib.cpab_transform_data_forward(2, 1, 2, ins, outs, 50, 2, 2, 1, 0, p, p, p, p, p, None,
                                         p, None)
    assert rc == 1 and "seed_grad" in _err(lib)
    rc = lib.cpab_transform_data_backward(2, 1, 2, ins, outs, 50, 2, 2, 1, 0, p, None, p, p, p, p,
                                          0, None, None, None, p, None, None, p, 1 << 30, None)
    assert rc == 1 and "seed_grad" in _err(lib)
    rc = lib.cpab_transform_data_backward(2, 1, 1, ins, outs, 50, 2, 2, 1, 0, p, None, None, p, p,
                                          p, 0, None, None, None, p, None, None, p, 1 << 30, None)
    assert rc == 1 and "final_points" in _err(lib)
    rc = lib.cpab_transform_data_backward(2, 1, 1, ins, outs, 50, 2, 2, 1, 0, p, None, p, p, p, p,
                                          0, None, None, None, p, None, p, p, 1 << 30, None)
    assert rc == 1 and "final_points" in _err(lib)


def test_missing_library_raises(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        _native.load_library(str(tmp_path / "nope.so"))


def test_chain_validation():
    _run_without_gpu("_check_chain_validation")


def _check_chain_validation():
    lib = _native.load_library()
    p = ctypes.c_void_p(16)
    rc = lib.cpab_chain_forward(2, 10, 1, 0, 0, 50, 4, 4, 1, 0, p, p, p, p, None, None)
    assert rc == 1 and "n_stages" in _err(lib)
    rc = lib.cpab_chain_backward(2, 10, 1, 0, 3, 50, 4, 4, 1, 0, p, None, p, p, 0, None, None,
                                 None, p, None, None, None, 0, None)
    assert rc == 1 and "stage_points" in _err(lib)
    rc = lib.cpab_chain_backward(2, 10, 1, 0, 5000, 50, 4, 4, 1, 0, p, p, p, p, 0, None, None,
                                 None, p, None, None, None, 0, None)
    assert rc == 1 and "n_stages" in _err(lib)
    # a projection needs B's tables
    rc = lib.cpab_backward_project(2, 10, 1, 0, 50, 4, 4, 1, 0, p, p, p, 5, None, None, None, p,
                                   p, None, None, 0, None)
    assert rc == 1 and "col_ptr" in _err(lib)
    assert lib.cpab_chain_backward_workspace_size(2, 10, 1, 0, 64) == 0


def test_misaligned_tables_rejected():
    _run_without_gpu("_check_misaligned_tables_rejected")


def _check_misaligned_tables_rejected():
    lib = _native.load_library()
    p = ctypes.c_void_p(64)
    bad = ctypes.c_void_p(68)  # float-aligned, not 16-byte aligned
    rc = lib.cpab_forward(2, 10, 1, 0, 50, 4, 4, 1, 0, p, p, bad, p, None)
    assert rc == 1 and "aligned" in _err(lib)
    rc = lib.cpab_expm(2, 4, 0.02, bad, p, None)
    assert rc == 1 and "aligned" in _err(lib)


def test_deterministic_toggle_is_per_thread():
    # cpab_set_deterministic sets the calling thread's mode only (no HIP call);
    # Native.deterministic restores the previous mode on exit.
    import threading
    lib = _native.load_library()
    assert lib.cpab_deterministic() == 0
    lib.cpab_set_deterministic(7)
    try:
        assert lib.cpab_deterministic() == 1
        seen = []
        t = threading.Thread(target=lambda: seen.append(lib.cpab_deterministic()))
        t.start()
        t.join()
        assert seen == [0]
    finally:
        lib.cpab_set_deterministic(0)
    assert lib.cpab_deterministic() == 0
    nat = _native.Native()
    with nat.deterministic(True):
        assert lib.cpab_deterministic() == 1
        with nat.deterministic(False):
            assert lib.cpab_deterministic() == 0
        assert lib.cpab_deterministic() == 1
    assert lib.cpab_deterministic() == 0
    with pytest.raises(ValueError):
        with nat.deterministic(True):
            raise ValueError("inside")
    assert lib.cpab_deterministic() == 0


def test_data_workspace_size_follows_the_mode():
    # The deterministic grad_data's extra workspace: none in the default mode,
    # a 64-bit sum per grad_data element in the deterministic one (no HIP call).
    lib = _native.load_library()
    ins = (ctypes.c_int64 * 2)(30, 26)
    assert lib.cpab_transform_data_backward_data_workspace_size(2, 4, 3, ins) == 0
    lib.cpab_set_deterministic(1)
    try:
        n = lib.cpab_transform_data_backward_data_workspace_size(2, 4, 3, ins)
        assert 4 * 3 * 30 * 26 * 8 <= n <= 4 * 3 * 30 * 26 * 8 + 4096
        assert lib.cpab_transform_data_backward_data_workspace_size(4, 4, 3, ins) == 0
        assert lib.cpab_transform_data_backward_data_workspace_size(2, 4, 0, ins) == 0
    finally:
        lib.cpab_set_deterministic(0)


def test_interp_workspace_size_follows_the_mode():
    lib = _native.load_library()
    ins = (ctypes.c_int64 * 3)(9, 8, 10)
    assert lib.cpab_interp_backward_workspace_size(3, 2, 3, ins) == 0
    lib.cpab_set_deterministic(1)
    try:
        n = lib.cpab_interp_backward_workspace_size(3, 2, 3, ins)
        assert 2 * 3 * 720 * 8 <= n <= 2 * 3 * 720 * 8 + 4096
    finally:
        lib.cpab_set_deterministic(0)


def test_deterministic_interp_limits():
    _run_without_gpu("_check_deterministic_interp_limits")


def _check_deterministic_interp_limits():
    lib = _native.load_library()
    p = ctypes.c_void_p(256)
    lib.cpab_set_deterministic(1)
    try:
        ins = (ctypes.c_int64 * 2)(8, 8)
        big = (ctypes.c_int64 * 2)(1 << 16, 1 << 15)   # 2^31 output points
        rc = lib.cpab_interp_backward_ws(2, 1, 1, ins, big, p, p, p, None, p, p, 1 << 20, None)
        assert rc == 1 and "2^31" in _err(lib)
        small = (ctypes.c_int64 * 2)(2, 2)
        rc = lib.cpab_interp_backward_ws(2, 70000, 1, ins, small, p, p, p, None, p, p, 1 << 30, None)
        assert rc == 1 and "65536" in _err(lib)
        # too small a workspace is rejected before anything is enqueued
        rc = lib.cpab_interp_backward_ws(2, 2, 1, ins, small, p, p, p, None, p, p, 16, None)
        assert rc == 1 and "workspace too small" in _err(lib)
    finally:
        lib.cpab_set_deterministic(0)
