"""ctypes binding of libbmx.so (the C ABI declared in include/bmx.h).

The library is built in-tree (``make -C base-mlx_amd``) to
``base-mlx_amd/lib/libbmx.so``.  There is no fallback: if the library is
missing, every call raises :class:`BmxNotBuilt`.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "lib", "libbmx.so"))

BMX_OK = 0
BMX_E_ARG = -1
BMX_E_SHAPE = -2
BMX_E_UNSUPPORTED = -3
BMX_E_KV_CAPACITY = -4
BMX_E_ALLOC = -5
BMX_E_ALIGN = -6

_ERR_NAMES = {
    BMX_E_ARG: "BMX_E_ARG",
    BMX_E_SHAPE: "BMX_E_SHAPE",
    BMX_E_UNSUPPORTED: "BMX_E_UNSUPPORTED",
    BMX_E_KV_CAPACITY: "BMX_E_KV_CAPACITY",
    BMX_E_ALLOC: "BMX_E_ALLOC",
    BMX_E_ALIGN: "BMX_E_ALIGN",
}


class BmxNotBuilt(RuntimeError):
    """libbmx.so is not present: build it with ``make -C base-mlx_amd``."""


class BmxError(RuntimeError):
    """A non-zero return code from the C ABI (mirrors Error::Inference)."""

    def __init__(self, code: int, message: str):
        self.code = code
        name = _ERR_NAMES.get(code, f"hipError_t {code}" if code > 0 else str(code))
        super().__init__(f"{name}: {message}")


_lock = threading.Lock()
_lib = None

c_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_u64 = ctypes.c_uint64
c_f = ctypes.c_float

# name -> (restype, argtypes); every symbol declared in include/bmx.h
SIGNATURES = {
    "bmx_last_error": (ctypes.c_char_p, []),
    "bmx_abi_version": (c_int, []),
    "bmx_qmatmul_affine": (c_int, [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_p]),
    "bmx_qmatmul_workspace_bytes": (ctypes.c_size_t, [c_i64, c_i64, c_i64]),
    "bmx_qmatmul_affine_noalloc": (c_int, [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_p]),
    "bmx_qmatmul_affine_ws": (c_int, [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_p,
                                      ctypes.c_size_t, c_p]),
    "bmx_dequantize_affine": (c_int, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_int, c_int, c_p]),
    "bmx_dequant_gather": (c_int, [c_p, c_i64, c_i64, c_p, c_p, c_p, c_p, c_i64, c_int, c_int, c_p]),
    "bmx_init_qlinear": (c_int, [c_u64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p]),
    "bmx_fill_normal_bf16": (c_int, [c_u64, c_i64, c_f, c_p, c_p]),
    "bmx_rms_norm": (c_int, [c_p, c_p, c_p, c_i64, c_i64, c_f, c_p]),
    "bmx_rope": (c_int, [c_p, c_p, c_i64, c_i64, c_i64, c_f, c_i64, c_p]),
    "bmx_slice_update": (c_int, [c_p, c_int, c_p, c_p, c_p, c_p, c_p, c_p]),
    "bmx_qk_norm_rope_kv": (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int,
                                    c_int, c_f, c_f, c_p]),
    "bmx_attention_gqa": (c_int, [c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_int, c_f, c_p,
                                  ctypes.c_size_t, c_p]),
    "bmx_attention_workspace_bytes": (ctypes.c_size_t, [c_int, c_int]),
    "bmx_qwen3_config_from_json": (c_int, [ctypes.c_char_p, c_p]),
    "bmx_qwen3_load": (c_int, [ctypes.c_char_p, c_int, c_p]),
    "bmx_gather_qmm": (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                               c_int, c_p]),
    "bmx_gather_qmm_indexed": (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_int, c_int, c_p]),
    "bmx_qk_norm_rope_kv_attention": (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_int,
                                              c_int, c_int, c_f, c_f, c_f, c_p, ctypes.c_size_t, c_p]),
    "bmx_argmax_rows": (c_int, [c_p, c_i64, c_i64, c_p, c_p]),
    "bmx_silu_mul": (c_int, [c_p, c_p, c_p, c_i64, c_p]),
    "bmx_add": (c_int, [c_p, c_p, c_p, c_i64, c_p]),
    "bmx_qwen3_create_random": (c_int, [c_p, c_u64, ctypes.c_double, c_int, c_p]),
    "bmx_qwen3_destroy": (None, [c_p]),
    "bmx_qwen3_qlinear": (c_int, [c_p, c_int, c_int, c_p, c_p, c_p, c_p, c_p]),
    "bmx_kv_create": (c_int, [c_p, c_int, c_p]),
    "bmx_kv_destroy": (None, [c_p]),
    "bmx_kv_seq_len": (c_int, [c_p]),
    "bmx_kv_capacity": (c_int, [c_p]),
    "bmx_kv_reset": (None, [c_p]),
    "bmx_kv_truncate": (None, [c_p, c_int]),
    "bmx_kv_data": (c_p, [c_p]),
    "bmx_kv_fill_synthetic": (c_int, [c_p, c_u64, c_int, c_p]),
    "bmx_qwen3_forward": (c_int, [c_p, c_p, c_p, c_int, c_int, c_p, c_p]),
    "bmx_qwen3_decode_step": (c_int, [c_p, c_p, ctypes.c_uint32, c_p, c_p, c_p]),
    "bmx_generate_greedy": (c_int, [c_p, c_p, c_p, c_int, c_int, c_p, c_int, c_p, c_p, c_p]),
    "bmx_decode_greedy": (c_int, [c_p, c_p, ctypes.c_uint32, c_int, c_p, c_int, c_p, c_p, c_p]),
    "bmx_speculative_generate": (c_int, [c_p, c_p, c_p, c_p, c_p, c_int, c_int, c_int, c_p, c_int, c_p, c_p, c_p,
                                         c_p]),
}


def load():
    """Load libbmx.so once and attach signatures; raise if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise BmxNotBuilt(f"{LIB_PATH} not found; run `make -C base-mlx_amd`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    return load().bmx_last_error().decode("utf-8", "replace")


def check(rc: int) -> None:
    if rc != 0:
        raise BmxError(rc, last_error())


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
