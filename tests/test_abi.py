"""The C ABI library builds for gfx950, loads, and exports every declared symbol.

CPU-only: no compute call is made here.
"""
import re
from pathlib import Path

import pytest

from tatara_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "tatara_hip.h").read_text()
    return sorted(set(re.findall(r"^TATARA_API\s+[\w\s\*]+?\b(tatara_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 25
    assert "tatara_trainer_train_step" in syms and "tatara_op_sparse_ft_forward" in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_covers_header():
    assert set(declared_symbols()) <= set(_lib.SIGNATURES), set(declared_symbols()) - set(_lib.SIGNATURES)


def test_library_is_built_for_gfx950_only():
    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert b"amdgcn-amd-amdhsa--" + other not in data


def test_version_and_error_strings():
    lib = _lib.load()
    assert b"gfx950" in lib.tatara_version()
    assert lib.tatara_last_error() is not None


def test_invalid_arguments_fail_loudly_without_gpu_work():
    import ctypes as C

    lib = _lib.load()
    # a null config is rejected before any device call
    assert lib.tatara_trainer_create(None, None) == -3
    assert b"invalid argument" in lib.tatara_last_error()
    # step >= 1 precondition of the RAdam pre-compute
    ss, dn = C.c_float(), C.c_int32()
    assert lib.tatara_radam_step_size_denom(0, 0.9, 0.999, 5.0, C.byref(ss), C.byref(dn)) == -3


def test_radam_host_precompute_matches_oracle():
    import ctypes as C

    from oracle import ffi

    lib = _lib.load()
    for step in (1, 2, 5, 6, 7, 100, 1000, 123456):
        for beta1 in (0.9, 0.99):
            ss, dn = C.c_float(), C.c_int32()
            assert lib.tatara_radam_step_size_denom(step, beta1, 0.999, 5.0, C.byref(ss), C.byref(dn)) == 0
            ess, edn = ffi.radam_step_size_denom(step, beta1, 0.999, 5.0)
            assert (ss.value, dn.value) == (ess, edn)


def test_quantise_noalloc_rejects_tables_beyond_its_scratch():
    """The allocation-free quantiser refuses more than 2^28 values (65536 tiles of
    4096) before any device call: the pointers are never touched (CPU only)."""
    import ctypes as C

    lib = _lib.load()
    n = C.c_uint64()
    fake = C.c_void_p(256)
    st = lib.tatara_op_quantise_ft_noalloc(fake, 1 << 20, 257, 0, 127.0, 1, fake, 1 << 40, C.byref(n))
    assert st == -3 and b"static scratch" in lib.tatara_last_error()
    assert n.value == 0


def test_runtime_surface_rejects_bad_arguments_without_gpu_work():
    """Null outputs, unknown event flags, and an image that is not a code
    object are refused before any device call (CPU only)."""
    import ctypes as C

    lib = _lib.load()
    assert lib.tatara_stream_create(0, None) == -3
    assert lib.tatara_event_create(0, 0, None) == -3
    h = C.c_void_p()
    assert lib.tatara_event_create(0, 4, C.byref(h)) == -3 and h.value is None
    assert b"event flags" in lib.tatara_last_error()
    junk = b"not a code object at all"
    assert lib.tatara_module_load_image(0, junk, len(junk), C.byref(h)) == -3
    assert b"code object" in lib.tatara_last_error()
    assert lib.tatara_module_load_image(0, None, 0, C.byref(h)) == -3
    grid = (C.c_uint32 * 3)(1, 1, 1)
    assert lib.tatara_module_launch(None, b"k", None, grid, grid, 0, None) == -3
    assert lib.tatara_host_alloc_pinned(16, None) == -3
    # destroying a null handle is a no-op
    assert lib.tatara_stream_destroy(None) == 0 and lib.tatara_event_destroy(None) == 0
    assert lib.tatara_module_destroy(None) == 0


def test_launch_geometry_helpers():
    from tatara_amd import runtime as rt

    assert rt.grid_dim_1d(0) == (1, 1, 1) and rt.grid_dim_1d(256) == (1, 1, 1)
    assert rt.grid_dim_1d(257) == (2, 1, 1) and rt.grid_dim_1d(1000, 128) == (8, 1, 1)
    cfg = rt.LaunchConfig.for_num_elems(1000)
    assert cfg.grid_dim == (4, 1, 1) and cfg.block_dim == (256, 1, 1) and cfg.shared_mem_bytes == 0


def test_selftest_code_object_is_built_for_gfx950():
    img = (ROOT / "tests" / "kernels" / "runtime_selftest.hsaco").read_bytes()
    assert img.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or img.startswith(b"\x7fELF")
    assert b"gfx950" in img and b"selftest_axpy" in img
