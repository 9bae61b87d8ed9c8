"""The C-ABI library loads and exports every symbol include/bmx.h declares,
and its host-side argument checks return the documented codes (no GPU
work is issued by any call here)."""
import ctypes
import os
import re

import pytest

import bmx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "bmx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bmx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "bmx_qmatmul_affine" in syms and "bmx_last_error" in syms
    # the Python binding knows the signature of every declared entry point
    assert sorted(bmx.SIGNATURES) == syms


def test_library_exports_every_declared_symbol():
    lib = bmx.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert lib.bmx_abi_version() >> 16 == 2


def _null():
    return ctypes.c_void_p(0)


def _fake(n=0x1000):
    # never dereferenced: every call below fails its host-side checks first
    return ctypes.c_void_p(n)


def test_qmatmul_rejects_unsupported_format():
    lib = bmx.load()
    rc = lib.bmx_qmatmul_affine(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 64, 64, 1, 64, 3, _null())
    assert rc == bmx.BMX_E_UNSUPPORTED
    assert "bits=4" in bmx.last_error()
    rc = lib.bmx_qmatmul_affine(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 64, 64, 1, 32, 4, _null())
    assert rc == bmx.BMX_E_UNSUPPORTED
    # transpose = false (W stored [K, N]) is not supported, as in the reference's use
    rc = lib.bmx_qmatmul_affine(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 64, 64, 0, 64, 4, _null())
    assert rc == bmx.BMX_E_UNSUPPORTED and "transpose" in bmx.last_error()


def test_qmatmul_rejects_bad_shapes_and_nulls():
    lib = bmx.load()
    assert lib.bmx_qmatmul_affine(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 64, 96, 1, 64, 4, _null()) == bmx.BMX_E_SHAPE
    assert lib.bmx_qmatmul_affine(_fake(), _fake(), _fake(), _fake(), _fake(), 1, 0, 64, 1, 64, 4, _null()) == bmx.BMX_E_SHAPE
    assert lib.bmx_qmatmul_affine(_null(), _fake(), _fake(), _fake(), _fake(), 1, 64, 64, 1, 64, 4, _null()) == bmx.BMX_E_ARG
    # misaligned x is refused before any launch
    assert lib.bmx_qmatmul_affine(_fake(0x1002), _fake(), _fake(), _fake(), _fake(), 1, 64, 64, 1, 64, 4, _null()) == bmx.BMX_E_ALIGN
    # M == 0 is a no-op
    assert lib.bmx_qmatmul_affine(_fake(), _fake(), _fake(), _fake(), _fake(), 0, 64, 64, 1, 64, 4, _null()) == 0


def test_dequant_rejects_bad_format():
    lib = bmx.load()
    assert lib.bmx_dequantize_affine(_fake(), _fake(), _fake(), _fake(), 4, 64, 64, 8, _null()) == bmx.BMX_E_UNSUPPORTED
    assert lib.bmx_dequant_gather(_fake(), 1, 10, _fake(), _fake(), _fake(), _fake(), 100, 64, 4, _null()) == bmx.BMX_E_SHAPE
    assert lib.bmx_init_qlinear(1, 4, 100, ctypes.c_float(1.0), _fake(), _fake(), _fake(), _null()) == bmx.BMX_E_SHAPE


def test_python_binding_raises_bmx_error():
    with pytest.raises(bmx.BmxError) as ei:
        bmx.call("bmx_qmatmul_affine", _fake(), _fake(), _fake(), _fake(), _fake(), 1, 64, 64, 1, 64, 3, _null())
    assert ei.value.code == bmx.BMX_E_UNSUPPORTED


def test_qmatmul_workspace_query_and_no_alloc_variant():
    """The workspace-taking GEMM reports a too-small (or missing) workspace
    as BMX_E_ARG before any launch instead of allocating one."""
    lib = bmx.load()
    assert lib.bmx_qmatmul_workspace_bytes(1, 4096, 2560) == 0
    assert lib.bmx_qmatmul_workspace_bytes(0, 4096, 2560) == 0
    assert lib.bmx_qmatmul_workspace_bytes(64, 1024, 100) == 0  # K not a multiple of 64
    # a small GEMM grid (8 tiles of 128 x 128) splits K = 2560: 5 splits of 8 groups
    need = lib.bmx_qmatmul_workspace_bytes(64, 1024, 2560)
    assert need == 5 * 64 * 1024 * 4
    args = (_fake(), _fake(), _fake(), _fake(), _fake(), 64, 1024, 2560, 1, 64, 4)
    assert lib.bmx_qmatmul_affine_ws(*args, _null(), 0, _null()) == bmx.BMX_E_ARG
    assert "workspace" in bmx.last_error()
    assert lib.bmx_qmatmul_affine_ws(*args, _fake(), need - 4, _null()) == bmx.BMX_E_ARG
    assert lib.bmx_qmatmul_affine_ws(*args, _fake(0x1004), need, _null()) == bmx.BMX_E_ALIGN
    assert lib.bmx_qmatmul_affine_ws(*args, _null(), 16, _null()) == bmx.BMX_E_ARG
    # transpose = false is refused here too
    targs = args[:8] + (0,) + args[9:]
    assert lib.bmx_qmatmul_affine_ws(*targs, _fake(), need, _null()) == bmx.BMX_E_UNSUPPORTED
