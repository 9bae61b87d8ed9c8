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
import os

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


def _qmatmul_args(x, w, scales, biases, group_size, bits):
    torch = _torch()
    _require_cuda(x, w, scales, biases)
    if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise BmxError(BMX_E_ARG, "x, scales and biases must be bfloat16")
    K = x.shape[-1]
    N = w.shape[0]
    if bits == 4 and w.shape[-1] * 8 != K:
        raise BmxError(BMX_E_SHAPE, f"w has {w.shape[-1]} words per row, K={K} needs {K // 8}")
    if scales.shape != biases.shape or scales.shape[0] != N or scales.shape[-1] * group_size != K:
        raise BmxError(BMX_E_SHAPE, f"scales/biases {tuple(scales.shape)} do not match N={N}, K={K}")
    return x.numel() // K, N, K


def quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4, out=None, stream=None):
    """y = x @ dequantize(w, scales, biases).T  (x [..., K] bf16, w [N, K/8] int32/uint32).

    transpose=False is rejected by the library (BMX_E_UNSUPPORTED), as the
    reference only ever passes True."""
    torch = _torch()
    M, N, K = _qmatmul_args(x, w, scales, biases, group_size, bits)
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    call("bmx_qmatmul_affine", _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out), M, N, K,
         1 if transpose else 0, group_size, bits, _stream(stream))
    return out


def qmatmul_workspace_bytes(M, N, K):
    """Bytes of split-K workspace quantized_matmul_ws needs for this shape."""
    return int(load().bmx_qmatmul_workspace_bytes(M, N, K))


def quantized_matmul_ws(x, w, scales, biases, workspace, transpose=True, group_size=64, bits=4, out=None,
                        stream=None):
    """quantized_matmul with the split-K partials in `workspace` (a CUDA tensor
    of at least qmatmul_workspace_bytes(M, N, K) bytes, or None when that is
    0); never allocates device memory in the library."""
    torch = _torch()
    M, N, K = _qmatmul_args(x, w, scales, biases, group_size, bits)
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    wp, wb = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel() * workspace.element_size())
    call("bmx_qmatmul_affine_ws", _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out), M, N, K,
         1 if transpose else 0, group_size, bits, wp, wb, _stream(stream))
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


# ---------------------------------------------------------------------------
# ops around the matmul
# ---------------------------------------------------------------------------
def rms_norm(x, w, eps=1e-6, out=None, stream=None):
    """fast::rms_norm over the last axis (bf16)."""
    torch = _torch()
    _require_cuda(x, w)
    out = torch.empty_like(x) if out is None else out
    dim = x.shape[-1]
    call("bmx_rms_norm", _ptr(x), _ptr(w), _ptr(out), x.numel() // dim, dim, ctypes.c_float(eps), _stream(stream))
    return out


def rope(x, theta, offset, out=None, stream=None):
    """fast::rope(x [H, T, D], D, traditional=False, theta, 1.0, offset)."""
    torch = _torch()
    _require_cuda(x)
    H, T, D = x.shape
    out = torch.empty_like(x) if out is None else out
    call("bmx_rope", _ptr(x), _ptr(out), H, T, D, ctypes.c_float(theta), offset, _stream(stream))
    return out


def slice_update(src, update, start, stop, strides, stream=None):
    """mlx_ext::slice_update: src[start:stop:strides] = update, in place; returns src."""
    import numpy as np

    _require_cuda(src, update)
    nd = src.dim()
    arrs = [np.ascontiguousarray(a, np.int64) for a in (list(src.shape), start, stop, strides)]
    if any(a.size != nd for a in arrs):
        raise BmxError(BMX_E_ARG, "start/stop/strides must have one entry per axis")
    p = [a.ctypes.data_as(ctypes.c_void_p) for a in arrs]
    call("bmx_slice_update", _ptr(src), nd, p[0], _ptr(update), p[1], p[2], p[3], _stream(stream))
    return src


def qk_norm_rope_kv(q, k, v, q_norm, k_norm, k_cache, v_cache, offset, eps=1e-6, theta=1e6, stream=None):
    """Fused QK-norm + RoPE + KV write; returns q_out [Hq, M, 128]."""
    torch = _torch()
    _require_cuda(q, k, v, q_norm, k_norm, k_cache, v_cache)
    Hkv, cap, D = k_cache.shape
    M = q.shape[0]
    Hq = q.shape[-1] // D
    q_out = torch.empty(Hq, M, D, dtype=torch.bfloat16, device=q.device)
    call("bmx_qk_norm_rope_kv", _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(q_out), _ptr(k_cache),
         _ptr(v_cache), M, Hq, Hkv, D, cap, offset, ctypes.c_float(eps), ctypes.c_float(theta), _stream(stream))
    return q_out


def attention(q, k_cache, v_cache, offset, scale=None, use_workspace=True, workspace=None, stream=None):
    """GQA SDPA of q [Hq, M, D] over cache rows [0, offset + M); returns [M, Hq*D]."""
    torch = _torch()
    _require_cuda(q, k_cache, v_cache)
    Hq, M, D = q.shape
    Hkv, cap, _ = k_cache.shape
    scale = 1.0 / (D ** 0.5) if scale is None else scale
    out = torch.empty(M, Hq * D, dtype=torch.bfloat16, device=q.device)
    if use_workspace and workspace is None:
        workspace = attention_workspace(Hq, M, q.device)
    nbytes = workspace.numel() * 4 if use_workspace else 0
    call("bmx_attention_gqa", _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), Hq, Hkv, M, D, cap, offset,
         ctypes.c_float(scale), _ptr(workspace if use_workspace else None), nbytes, _stream(stream))
    return out


def attention_workspace(Hq, M, device="cuda"):
    """A zero-filled attention workspace (arrival counters + split partials)."""
    torch = _torch()
    nbytes = load().bmx_attention_workspace_bytes(Hq, M)
    return torch.zeros(max(nbytes // 4, 1), dtype=torch.float32, device=device)


def qk_norm_rope_kv_attention(q, k, v, q_norm, k_norm, k_cache, v_cache, offset, eps=1e-6, theta=1e6, scale=None,
                              workspace=None, stream=None):
    """Fused QK-norm + RoPE + KV write + GQA attention of M new tokens; returns [M, Hq*128]."""
    torch = _torch()
    _require_cuda(q, k, v, q_norm, k_norm, k_cache, v_cache)
    Hkv, cap, D = k_cache.shape
    M = q.shape[0]
    Hq = q.shape[-1] // D
    scale = 1.0 / (D ** 0.5) if scale is None else scale
    if workspace is None:
        workspace = attention_workspace(Hq, M, q.device)
    out = torch.empty(M, Hq * D, dtype=torch.bfloat16, device=q.device)
    call("bmx_qk_norm_rope_kv_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(k_cache),
         _ptr(v_cache), _ptr(out), M, Hq, Hkv, D, cap, offset, ctypes.c_float(eps), ctypes.c_float(theta),
         ctypes.c_float(scale), _ptr(workspace), workspace.numel() * 4, _stream(stream))
    return out


def gather_qmm(x, w, scales, biases, rhs_indices, x_bcast=1, out=None, stream=None):
    """mlx_ext::gather_qmm (transpose=true, gs 64, 4 bits, lhs_indices None):
    x [R / x_bcast, M, K] bf16, w [E, N, K/8] uint32 (int32 storage), scales /
    biases [E, N, K/64] bf16, rhs_indices [R] int32/uint32 on the device ->
    [R, M, N] bf16; route r uses x block r // x_bcast and expert rhs[r]."""
    torch = _torch()
    _require_cuda(x, w, scales, biases, rhs_indices)
    E, N = w.shape[0], w.shape[1]
    M, K = x.shape[-2], x.shape[-1]
    R = rhs_indices.numel()
    if x.numel() != (R // x_bcast) * M * K or R % x_bcast:
        raise BmxError(BMX_E_SHAPE, f"x holds {x.numel()} values; {R // x_bcast} blocks of [{M}, {K}] expected")
    if out is None:
        out = torch.empty(R, M, N, dtype=torch.bfloat16, device=x.device)
    call("bmx_gather_qmm", _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(rhs_indices), _ptr(out), R, x_bcast,
         E, M, N, K, 64, 4, _stream(stream))
    return out


def gather_qmm_indexed(x, w, scales, biases, lhs_indices=None, rhs_indices=None, transpose=True, group_size=64,
                       bits=4, sorted_indices=False, out=None, stream=None):
    """mlx_ext::gather_qmm with both index arrays (mlx_ext.rs:66-117): x [B, M,
    K] bf16 (B row blocks), w [E, N, K/8], scales / biases [E, N, K/64];
    lhs_indices / rhs_indices [R] int32/uint32 on the device or None ->
    [R, M, N] bf16.  Route r uses x block lhs[r] (None: r // (R // B)) and
    expert rhs[r] (None: r, with R == E); R is the length of whichever
    index array is given (both: equal lengths)."""
    torch = _torch()
    _require_cuda(x, w, scales, biases, *[t for t in (lhs_indices, rhs_indices) if t is not None])
    E, N = w.shape[0], w.shape[1]
    M, K = x.shape[-2], x.shape[-1]
    B = x.numel() // (M * K)
    lens = {t.numel() for t in (lhs_indices, rhs_indices) if t is not None}
    if len(lens) > 1:
        raise BmxError(BMX_E_SHAPE, f"lhs_indices and rhs_indices differ in length: {sorted(lens)}")
    R = lens.pop() if lens else E
    if out is None:
        out = torch.empty(R, M, N, dtype=torch.bfloat16, device=x.device)
    call("bmx_gather_qmm_indexed", _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(lhs_indices),
         _ptr(rhs_indices), _ptr(out), R, B, E, M, N, K, int(bool(transpose)), group_size, bits,
         int(bool(sorted_indices)), _stream(stream))
    return out


def argmax_rows(x, stream=None):
    torch = _torch()
    _require_cuda(x)
    n = x.shape[-1]
    out = torch.empty(x.numel() // n, dtype=torch.int32, device=x.device)
    call("bmx_argmax_rows", _ptr(x), x.numel() // n, n, _ptr(out), _stream(stream))
    return out


def silu_mul(g, u, stream=None):
    torch = _torch()
    _require_cuda(g, u)
    y = torch.empty_like(g)
    call("bmx_silu_mul", _ptr(g), _ptr(u), _ptr(y), g.numel(), _stream(stream))
    return y


def add(a, b, stream=None):
    torch = _torch()
    _require_cuda(a, b)
    y = torch.empty_like(a)
    call("bmx_add", _ptr(a), _ptr(b), _ptr(y), a.numel(), _stream(stream))
    return y


# ---------------------------------------------------------------------------
# Qwen3 model / KV cache / generation (host mirror of the reference's
# Qwen3, KvCache, LoadedModel::generate_text and speculative::generate)
# ---------------------------------------------------------------------------
class Qwen3Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("hidden", "inter", "layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "tied",
                 "group_size", "bits")] + [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


def qwen3_config(hidden, inter, layers, n_heads, n_kv_heads, head_dim=128, vocab=151936, tied=1, eps=1e-6,
                 rope_theta=1e6):
    return Qwen3Config(hidden, inter, layers, n_heads, n_kv_heads, head_dim, vocab, tied, 64, 4, eps, rope_theta)


def qwen3_config_from_json(path):
    """ModelConfig::from_path: a config.json -> Qwen3Config (host only)."""
    cfg = Qwen3Config()
    call("bmx_qwen3_config_from_json", os.fsencode(path), ctypes.byref(cfg))
    return cfg


# Qwen3-shaped configurations of the benchmark workloads
QWEN3_0_6B = dict(hidden=1024, inter=3072, layers=28, n_heads=16, n_kv_heads=8)
QWEN3_4B = dict(hidden=2560, inter=9728, layers=36, n_heads=32, n_kv_heads=8)
QWEN3_8B = dict(hidden=4096, inter=12288, layers=36, n_heads=32, n_kv_heads=8)
QWEN3_32B = dict(hidden=5120, inter=25600, layers=64, n_heads=64, n_kv_heads=8, tied=0)

_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.restype = ctypes.c_int
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _HIP


def device_to_numpy(ptr, shape, dtype):
    """Copy `shape` elements of `dtype` at device address `ptr` into a numpy array."""
    import numpy as np

    out = np.empty(shape, dtype)
    rc = _hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), out.nbytes, 2)
    if rc != 0:
        raise BmxError(rc, "hipMemcpy device->host failed")
    return out


class KvCache:
    """bmx_kv_cache: [layers, 2, n_kv_heads, capacity, 128] bf16 on the GPU."""

    def __init__(self, model, capacity):
        self.model = model
        h = ctypes.c_void_p()
        call("bmx_kv_create", model.h, capacity, ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            load().bmx_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def seq_len(self):
        return load().bmx_kv_seq_len(self.h)

    @property
    def capacity(self):
        return load().bmx_kv_capacity(self.h)

    def reset(self):
        load().bmx_kv_reset(self.h)

    def truncate(self, target):
        load().bmx_kv_truncate(self.h, target)

    def fill_synthetic(self, seed, seq_len, stream=None):
        call("bmx_kv_fill_synthetic", self.h, ctypes.c_uint64(seed), seq_len, _stream(stream))

    def layer_numpy(self, layer, kv):
        """Host copy of K (kv=0) or V (kv=1) of one layer: [n_kv_heads, capacity, 128] uint16."""
        import numpy as np

        c = self.model.cfg
        cap = self.capacity
        n = c.n_kv_heads * cap * c.head_dim
        base = load().bmx_kv_data(self.h) + 2 * n * (2 * layer + kv)
        return device_to_numpy(base, (c.n_kv_heads, cap, c.head_dim), np.uint16)


class Qwen3:
    """Random-init Qwen3 on the GPU behind the C ABI (bmx_qwen3_*)."""

    def __init__(self, cfg, seed, sigma=0.02, max_tokens=256):
        self.cfg = cfg
        h = ctypes.c_void_p()
        call("bmx_qwen3_create_random", ctypes.byref(cfg), ctypes.c_uint64(seed), ctypes.c_double(sigma), max_tokens,
             ctypes.byref(h))
        self.h = h
        self.max_tokens = max_tokens

    @classmethod
    def load(cls, path, max_tokens=256):
        """Qwen3::load: an MLX checkpoint directory (config.json + *.safetensors)."""
        self = cls.__new__(cls)
        self.cfg = qwen3_config_from_json(os.path.join(path, "config.json"))
        h = ctypes.c_void_p()
        call("bmx_qwen3_load", os.fsencode(path), max_tokens, ctypes.byref(h))
        self.h = h
        self.max_tokens = max_tokens
        return self

    def close(self):
        if self.h:
            load().bmx_qwen3_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_cache(self, capacity):
        return KvCache(self, capacity)

    def qlinear_numpy(self, layer, slot):
        """Host copies (w uint32, s uint16, b uint16) of one projection."""
        import numpy as np

        w, s, b = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        N, K = ctypes.c_int(), ctypes.c_int()
        call("bmx_qwen3_qlinear", self.h, layer, slot, ctypes.byref(w), ctypes.byref(s), ctypes.byref(b),
             ctypes.byref(N), ctypes.byref(K))
        n, k = N.value, K.value
        return (device_to_numpy(w.value, (n, k // 8), np.uint32), device_to_numpy(s.value, (n, k // 64), np.uint16),
                device_to_numpy(b.value, (n, k // 64), np.uint16))

    def forward(self, cache, tokens, all_logits=False, stream=None):
        """Qwen3::forward / forward_multi: logits bf16 [vocab] or [M, vocab] (torch, on the GPU)."""
        import numpy as np

        torch = _torch()
        toks = np.ascontiguousarray(tokens, np.uint32)
        M = toks.size
        out = torch.empty(M if all_logits else 1, self.cfg.vocab, dtype=torch.bfloat16, device="cuda")
        call("bmx_qwen3_forward", self.h, cache.h, toks.ctypes.data_as(ctypes.c_void_p), M, int(all_logits), _ptr(out),
             _stream(stream))
        return out if all_logits else out[0]

    def decode_step(self, cache, token, want_logits=False, stream=None):
        torch = _torch()
        nxt = ctypes.c_uint32()
        out = torch.empty(self.cfg.vocab, dtype=torch.bfloat16, device="cuda") if want_logits else None
        call("bmx_qwen3_decode_step", self.h, cache.h, ctypes.c_uint32(int(token)), ctypes.byref(nxt), _ptr(out),
             _stream(stream))
        return (nxt.value, out) if want_logits else nxt.value

    def generate_greedy(self, cache, prompt, max_new, eos=(151645, 151643), stream=None):
        import numpy as np

        p = np.ascontiguousarray(prompt, np.uint32)
        e = np.ascontiguousarray(eos, np.uint32)
        out = np.empty(max_new, np.uint32)
        n = ctypes.c_int()
        call("bmx_generate_greedy", self.h, cache.h, p.ctypes.data_as(ctypes.c_void_p), p.size, max_new,
             e.ctypes.data_as(ctypes.c_void_p), e.size, out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n),
             _stream(stream))
        return out[: n.value]

    def decode_greedy(self, cache, token, max_new, eos=(151645, 151643), stream=None):
        """The greedy decode loop alone (engine.rs:103-115), continuing `cache`
        from `token`, the token its prefill picked: returns the emitted tokens
        (token first), at most max_new, stopping before an eos token."""
        import numpy as np

        e = np.ascontiguousarray(eos, np.uint32)
        out = np.empty(max_new, np.uint32)
        n = ctypes.c_int()
        try:
            call("bmx_decode_greedy", self.h, cache.h, ctypes.c_uint32(int(token)), max_new,
                 e.ctypes.data_as(ctypes.c_void_p), e.size, out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n),
                 _stream(stream))
        except BmxError as err:
            err.tokens = out[: n.value]
            raise
        return out[: n.value]


def speculative_generate(target, tcache, draft, dcache, prompt, max_new, spec_k=5, eos=(151645, 151643), stream=None):
    import numpy as np

    p = np.ascontiguousarray(prompt, np.uint32)
    e = np.ascontiguousarray(eos, np.uint32)
    out = np.empty(max_new + spec_k, np.uint32)
    n = ctypes.c_int()
    stats = np.zeros(3, np.int64)
    call("bmx_speculative_generate", target.h, tcache.h, draft.h, dcache.h, p.ctypes.data_as(ctypes.c_void_p), p.size,
         max_new, spec_k, e.ctypes.data_as(ctypes.c_void_p), e.size, out.ctypes.data_as(ctypes.c_void_p),
         ctypes.byref(n), stats.ctypes.data_as(ctypes.c_void_p), _stream(stream))
    return out[: n.value], stats
