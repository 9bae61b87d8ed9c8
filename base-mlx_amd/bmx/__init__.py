"""bmx -- MI355X-native MLX-format 4-bit affine quantized matmul.

Python host binding of ``libbmx.so``.  Device buffers are torch tensors
(torch is used only for device memory and streams); every computation runs
in the HIP kernels behind the C ABI of ``include/bmx.h``.  The names and
argument meanings mirror the reference's operator surface:

* :func:`quantized_matmul` -- ``mlx_rs::ops::quantized_matmul(x, w, scales,
  biases, transpose=true, group_size, bits)``
  (crates/base-mlx-core/src/model/qwen3.rs:30-41)
* :func:`dequantize` -- ``mlx_rs::ops::dequantize`` (qwen3.rs:75)

Errors surface as :class:`BmxError` (the reference maps them to
``Error::Inference(String)``, qwen3.rs:40).
"""
from __future__ import annotations

import ctypes

from ._lib import (  # noqa: F401
    BMX_E_ALIGN,
    BMX_E_ALLOC,
    BMX_E_ARG,
    BMX_E_KV_CAPACITY,
    BMX_E_SHAPE,
    BMX_E_UNSUPPORTED,
    LIB_PATH,
    SIGNATURES,
    BmxError,
    BmxNotBuilt,
    call,
    check,
    last_error,
    load,
)

IRWIN4_STD = 37837.226523565  # std of the sum of four uniform 16-bit integers


def _torch():
    import torch

    return torch


def sigma_to_c(sigma: float) -> float:
    """Scale c such that the generator's deviates have standard deviation sigma."""
    import numpy as np

    return float(np.float32(sigma / IRWIN4_STD))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(stream=None):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _require_cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise BmxError(BMX_E_ARG, "tensors must live on the GPU")
        if not t.is_contiguous():
            raise BmxError(BMX_E_ARG, "tensors must be contiguous")


def quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4, out=None, stream=None):
    """y = x @ dequantize(w, scales, biases).T  (x [..., K] bf16, w [N, K/8] int32/uint32)."""
    torch = _torch()
    if not transpose:
        raise BmxError(BMX_E_UNSUPPORTED, "only transpose=True is implemented (the reference's only use)")
    _require_cuda(x, w, scales, biases)
    if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise BmxError(BMX_E_ARG, "x, scales and biases must be bfloat16")
    K = x.shape[-1]
    N = w.shape[0]
    if bits == 4 and w.shape[-1] * 8 != K:
        raise BmxError(BMX_E_SHAPE, f"w has {w.shape[-1]} words per row, K={K} needs {K // 8}")
    if scales.shape != biases.shape or scales.shape[0] != N or scales.shape[-1] * group_size != K:
        raise BmxError(BMX_E_SHAPE, f"scales/biases {tuple(scales.shape)} do not match N={N}, K={K}")
    M = x.numel() // K
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    call("bmx_qmatmul_affine", _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out), M, N, K,
         group_size, bits, _stream(stream))
    return out


def dequantize(w, scales, biases, group_size=64, bits=4, stream=None):
    torch = _torch()
    _require_cuda(w, scales, biases)
    N, K = w.shape[0], w.shape[1] * 8
    out = torch.empty(N, K, dtype=torch.bfloat16, device=w.device)
    call("bmx_dequantize_affine", _ptr(w), _ptr(scales), _ptr(biases), _ptr(out), N, K, group_size, bits,
         _stream(stream))
    return out


def dequant_gather(ids, w, scales, biases, group_size=64, bits=4, stream=None):
    """QEmbedding::lookup: rows `ids` (int32, on device) of the quantized table, dequantized."""
    torch = _torch()
    _require_cuda(ids, w, scales, biases)
    if ids.dtype != torch.int32:
        raise BmxError(BMX_E_ARG, "ids must be int32")
    rows, K = w.shape[0], w.shape[1] * 8
    out = torch.empty(ids.numel(), K, dtype=torch.bfloat16, device=w.device)
    call("bmx_dequant_gather", _ptr(ids), ids.numel(), rows, _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
         K, group_size, bits, _stream(stream))
    return out


def init_qlinear(seed: int, N: int, K: int, sigma: float = 0.02, device="cuda", stream=None):
    """Seeded random-init MLX-format projection (w int32 [N, K/8], scales, biases bf16 [N, K/64])."""
    torch = _torch()
    w = torch.empty(N, K // 8, dtype=torch.int32, device=device)
    s = torch.empty(N, K // 64, dtype=torch.bfloat16, device=device)
    b = torch.empty(N, K // 64, dtype=torch.bfloat16, device=device)
    call("bmx_init_qlinear", ctypes.c_uint64(seed), N, K, ctypes.c_float(sigma_to_c(sigma)), _ptr(w), _ptr(s),
         _ptr(b), _stream(stream))
    return w, s, b


def fill_normal_bf16(seed: int, shape, sigma: float = 1.0, device="cuda", stream=None):
    torch = _torch()
    out = torch.empty(*shape, dtype=torch.bfloat16, device=device)
    call("bmx_fill_normal_bf16", ctypes.c_uint64(seed), out.numel(), ctypes.c_float(sigma_to_c(sigma)), _ptr(out),
         _stream(stream))
    return out
