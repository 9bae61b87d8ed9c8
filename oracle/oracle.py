"""numpy binding of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.  The product library never uses it.
bf16 arrays are numpy uint16 bit patterns; packed weights are uint32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
IRWIN4_STD = 37837.226523565

_lib = None
P = ctypes.c_void_p
I64 = ctypes.c_int64
INT = ctypes.c_int
U64 = ctypes.c_uint64
F = ctypes.c_float

_SIGS = {
    "orc_f2bf": (ctypes.c_uint16, [F]),
    "orc_bf2f": (F, [ctypes.c_uint16]),
    "orc_rand64": (U64, [U64, U64]),
    "orc_tensor_seed": (U64, [U64, INT, INT]),
    "orc_normal_at": (F, [U64, U64, F]),
    "orc_sigma_to_c": (F, [ctypes.c_double]),
    "orc_fill_normal_bf16": (None, [U64, I64, F, P]),
    "orc_fill_normal_f32": (None, [U64, I64, F, P]),
    "orc_fill_tokens": (None, [U64, I64, ctypes.c_uint32, P]),
    "orc_quantize_affine": (INT, [P, I64, I64, INT, INT, P, P, P]),
    "orc_init_qlinear": (None, [U64, I64, I64, F, P, P, P]),
    "orc_dequantize": (INT, [P, P, P, I64, I64, INT, INT, P]),
    "orc_dequant_gather": (INT, [P, I64, I64, P, P, P, I64, INT, INT, P]),
    "orc_qmatmul": (INT, [P, P, P, P, P, I64, I64, I64, INT, INT]),
    "orc_gather_qmm": (INT, [P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, INT, INT]),
    "orc_qmatmul_f64": (INT, [P, P, P, P, P, I64, I64, I64, INT, INT]),
    "orc_qmm_dequant": (INT, [P, P, P, P, P, I64, I64, I64, INT, INT]),
    "orc_qlinear": (INT, [P, P, P, P, P, I64, I64, I64, INT, INT]),
    "orc_rms_norm": (None, [P, P, P, I64, I64, F]),
    "orc_rope": (None, [P, P, I64, I64, I64, F, I64]),
    "orc_slice_update": (INT, [P, INT, P, P, P, P, P]),
    "orc_sdpa": (None, [P, P, P, P, I64, I64, I64, I64, I64, I64, I64, INT, F]),
    "orc_silu_mul": (None, [P, P, P, I64]),
    "orc_add": (None, [P, P, P, I64]),
    "orc_argmax_rows": (None, [P, I64, I64, P]),
    "orc_qwen3_create_random": (P, [P, U64, ctypes.c_double]),
    "orc_qwen3_free": (None, [P]),
    "orc_qwen3_qlinear": (INT, [P, INT, INT, P, P, P, P, P]),
    "orc_qwen3_norm": (P, [P, INT, INT]),
    "orc_kv_create": (P, [P, INT]),
    "orc_kv_free": (None, [P]),
    "orc_kv_seq_len": (INT, [P]),
    "orc_kv_capacity": (INT, [P]),
    "orc_kv_reset": (None, [P]),
    "orc_kv_truncate": (None, [P, INT]),
    "orc_kv_data": (P, [P]),
    "orc_kv_fill_synthetic": (None, [P, U64, INT]),
    "orc_qwen3_forward": (INT, [P, P, P, INT, INT, P]),
    "orc_generate_greedy": (INT, [P, P, P, INT, INT, P, INT, P, P]),
    "orc_speculative_generate": (INT, [P, P, P, P, P, INT, INT, INT, P, INT, P, P, P]),
    "orc_set_reverse_accumulation": (None, [INT]),
    "orc_num_threads": (INT, []),
    "orc_stream_triad_gbs": (ctypes.c_double, [I64, INT]),
}


def build():
    subprocess.run(["make", "-C", _HERE, "-s"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def num_threads():
    """OpenMP threads the oracle's parallel loops use."""
    return int(lib().orc_num_threads())


def stream_triad_gbs(n=1 << 26, reps=5):
    """Host memory bandwidth: best-of-`reps` STREAM triad over n doubles."""
    return float(lib().orc_stream_triad_gbs(n, reps))


class reversed_accumulation:
    """Context manager: inside it every fp32 reduction of the oracle (GEMV,
    GEMM, SDPA, RMSNorm) adds its terms in reverse order (the spread fp32
    summation order alone causes)."""

    def __enter__(self):
        lib().orc_set_reverse_accumulation(1)
        return self

    def __exit__(self, *exc):
        lib().orc_set_reverse_accumulation(0)
        return False


def _chk(rc):
    if rc != 0:
        raise RuntimeError(f"oracle error {rc}")


# ---- bf16 helpers (vectorised, numpy) --------------------------------------
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def sigma_to_c(sigma: float) -> float:
    return float(np.float32(sigma / IRWIN4_STD))


# ---- generator / format -------------------------------------------------------
def fill_normal_bf16(seed, n, sigma=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_fill_normal_bf16(seed, n, sigma_to_c(sigma), _p(out))
    return out


def fill_normal_f32(seed, n, sigma=1.0):
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(seed, n, sigma_to_c(sigma), _p(out))
    return out


def fill_tokens(seed, n, vocab):
    out = np.empty(n, np.uint32)
    lib().orc_fill_tokens(seed, n, vocab, _p(out))
    return out


def quantize(w: np.ndarray, gs=64, bits=4):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    wq = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // gs), np.uint16)
    b = np.empty((N, K // gs), np.uint16)
    _chk(lib().orc_quantize_affine(_p(w), N, K, gs, bits, _p(wq), _p(s), _p(b)))
    return wq, s, b


def init_qlinear(seed, N, K, sigma=0.02):
    wq = np.empty((N, K // 8), np.uint32)
    s = np.empty((N, K // 64), np.uint16)
    b = np.empty((N, K // 64), np.uint16)
    lib().orc_init_qlinear(seed, N, K, sigma_to_c(sigma), _p(wq), _p(s), _p(b))
    return wq, s, b


def dequantize(wq, s, b, gs=64, bits=4):
    N, K = wq.shape[0], wq.shape[1] * 8
    out = np.empty((N, K), np.uint16)
    _chk(lib().orc_dequantize(_p(wq), _p(s), _p(b), N, K, gs, bits, _p(out)))
    return out


def dequant_gather(ids, wq, s, b, gs=64, bits=4):
    ids = np.ascontiguousarray(ids, np.uint32)
    K = wq.shape[1] * 8
    out = np.empty((ids.size, K), np.uint16)
    _chk(lib().orc_dequant_gather(_p(ids), ids.size, wq.shape[0], _p(wq), _p(s), _p(b), K, gs, bits, _p(out)))
    return out


def qmatmul(x, wq, s, b, gs=64, bits=4):
    x = np.ascontiguousarray(x, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[0]
    y = np.empty((M, N), np.uint16)
    _chk(lib().orc_qmatmul(_p(x), _p(wq), _p(s), _p(b), _p(y), M, N, K, gs, bits))
    return y


def gather_qmm(x, wq, s, b, rhs, x_bcast=1, gs=64, bits=4):
    """Routed qmm: x [R / x_bcast, M, K], wq [E, N, K/8], rhs [R] -> [R, M, N]."""
    x = np.ascontiguousarray(x, np.uint16)
    wq = np.ascontiguousarray(wq, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    rhs = np.ascontiguousarray(rhs, np.uint32)
    E, N = wq.shape[0], wq.shape[1]
    M, K = x.shape[-2], x.shape[-1]
    R = rhs.size
    assert x.size == (R // x_bcast) * M * K
    y = np.empty((R, M, N), np.uint16)
    _chk(lib().orc_gather_qmm(_p(x), _p(wq), _p(s), _p(b), _p(rhs), _p(y), R, x_bcast, E, M, N, K, gs, bits))
    return y


def qmm_dequant(x, wq, s, b, gs=64, bits=4):
    """Matrix path: bf16-dequantized weights, fp32-accumulated x w^T."""
    x = np.ascontiguousarray(x, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[0]
    y = np.empty((M, N), np.uint16)
    _chk(lib().orc_qmm_dequant(_p(x), _p(wq), _p(s), _p(b), _p(y), M, N, K, gs, bits))
    return y


def qlinear(x, wq, s, b, gs=64, bits=4):
    """The product's dispatch: qmatmul for M <= 8 rows, qmm_dequant beyond."""
    x = np.ascontiguousarray(x, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[0]
    y = np.empty((M, N), np.uint16)
    _chk(lib().orc_qlinear(_p(x), _p(wq), _p(s), _p(b), _p(y), M, N, K, gs, bits))
    return y


def qmatmul_f64(x, wq, s, b, gs=64, bits=4):
    x = np.ascontiguousarray(x, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[0]
    y = np.empty((M, N), np.float64)
    _chk(lib().orc_qmatmul_f64(_p(x), _p(wq), _p(s), _p(b), _p(y), M, N, K, gs, bits))
    return y


def rms_norm(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, np.uint16)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(np.ascontiguousarray(w, np.uint16)), _p(y), x.size // dim, dim, eps)
    return y


def rope(x, theta, offset):
    """x: [H, T, D] bf16 bits."""
    x = np.ascontiguousarray(x, np.uint16)
    H, T, D = x.shape
    y = np.empty_like(x)
    lib().orc_rope(_p(x), _p(y), H, T, D, theta, offset)
    return y


def slice_update(src, update, start, stop, strides):
    shape = np.asarray(src.shape, np.int64)
    rc = lib().orc_slice_update(_p(src), src.ndim, _p(shape), _p(np.ascontiguousarray(update, np.uint16)),
                                _p(np.asarray(start, np.int64)), _p(np.asarray(stop, np.int64)),
                                _p(np.asarray(strides, np.int64)))
    return rc


def sdpa(q, k, v, L, offset, causal, scale, kv_stride=None):
    """q [Hq, M, D]; k, v [Hkv, stride, D]; returns [M, Hq*D] bf16 bits."""
    q = np.ascontiguousarray(q, np.uint16)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    Hq, M, D = q.shape
    Hkv = k.shape[0]
    stride = k.shape[1] if kv_stride is None else kv_stride
    out = np.empty((M, Hq * D), np.uint16)
    lib().orc_sdpa(_p(q), _p(k), _p(v), _p(out), Hq, Hkv, M, L, D, stride, offset, int(causal), scale)
    return out


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.uint16)
    y = np.empty_like(g)
    lib().orc_silu_mul(_p(g), _p(np.ascontiguousarray(u, np.uint16)), _p(y), g.size)
    return y


def argmax_rows(x):
    x = np.ascontiguousarray(x, np.uint16)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(rows, np.uint32)
    lib().orc_argmax_rows(_p(x), rows, n, _p(out))
    return out


# ---- Qwen3 --------------------------------------------------------------------
class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("hidden", "inter", "layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "tied",
                 "group_size", "bits")] + [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


def make_config(hidden, inter, layers, n_heads, n_kv_heads, head_dim=128, vocab=151936, tied=1,
                eps=1e-6, rope_theta=1e6):
    return Config(hidden, inter, layers, n_heads, n_kv_heads, head_dim, vocab, tied, 64, 4, eps, rope_theta)


class Qwen3:
    """Seeded random-init Qwen3 on the CPU (approx N(0, sigma) projections, norms 1)."""

    def __init__(self, cfg: Config, seed: int, sigma: float = 0.02):
        self.cfg = cfg
        self.h = lib().orc_qwen3_create_random(ctypes.byref(cfg), seed, sigma)
        if not self.h:
            raise MemoryError("oracle model allocation failed")

    def close(self):
        if self.h:
            lib().orc_qwen3_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def qlinear(self, layer, slot):
        w, s, b = P(), P(), P()
        N, K = INT(), INT()
        _chk(lib().orc_qwen3_qlinear(self.h, layer, slot, ctypes.byref(w), ctypes.byref(s), ctypes.byref(b),
                                     ctypes.byref(N), ctypes.byref(K)))
        n, k = N.value, K.value
        wa = np.ctypeslib.as_array(ctypes.cast(w, ctypes.POINTER(ctypes.c_uint32)), (n, k // 8))
        sa = np.ctypeslib.as_array(ctypes.cast(s, ctypes.POINTER(ctypes.c_uint16)), (n, k // 64))
        ba = np.ctypeslib.as_array(ctypes.cast(b, ctypes.POINTER(ctypes.c_uint16)), (n, k // 64))
        return wa, sa, ba

    def norm(self, layer, which):
        """Writable view of a norm weight (bf16 bits): layer -1 = final norm;
        which 0..3 = input, post-attention, q, k."""
        p = lib().orc_qwen3_norm(self.h, layer, which)
        if not p:
            raise IndexError((layer, which))
        n = self.cfg.head_dim if (layer >= 0 and which >= 2) else self.cfg.hidden
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint16)), (n,))

    def new_cache(self, capacity):
        return KvCache(self, capacity)

    def forward(self, cache, tokens, all_logits=False):
        tokens = np.ascontiguousarray(tokens, np.uint32)
        M = tokens.size
        out = np.empty((M if all_logits else 1, self.cfg.vocab), np.uint16)
        rc = lib().orc_qwen3_forward(self.h, cache.h, _p(tokens), M, int(all_logits), _p(out))
        if rc != 0:
            raise RuntimeError(f"oracle forward error {rc}")
        return out if all_logits else out[0]


class KvCache:
    def __init__(self, model: Qwen3, capacity: int):
        self.model = model
        self.h = lib().orc_kv_create(model.h, capacity)
        if not self.h:
            raise MemoryError("oracle KV allocation failed")

    def close(self):
        if self.h:
            lib().orc_kv_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def seq_len(self):
        return lib().orc_kv_seq_len(self.h)

    def reset(self):
        lib().orc_kv_reset(self.h)

    def truncate(self, t):
        lib().orc_kv_truncate(self.h, t)

    def fill_synthetic(self, seed, seq_len):
        lib().orc_kv_fill_synthetic(self.h, seed, seq_len)

    def data(self):
        c = self.model.cfg
        cap = lib().orc_kv_capacity(self.h)
        ptr = ctypes.cast(lib().orc_kv_data(self.h), ctypes.POINTER(ctypes.c_uint16))
        return np.ctypeslib.as_array(ptr, (c.layers, 2, c.n_kv_heads, cap, c.head_dim))


def generate_greedy(model, cache, prompt, max_new, eos=(151645, 151643)):
    prompt = np.ascontiguousarray(prompt, np.uint32)
    eos_a = np.asarray(eos, np.uint32)
    out = np.empty(max_new, np.uint32)
    n = INT()
    _chk(lib().orc_generate_greedy(model.h, cache.h, _p(prompt), prompt.size, max_new, _p(eos_a), eos_a.size,
                                   _p(out), ctypes.byref(n)))
    return out[: n.value]


def speculative_generate(target, tcache, draft, dcache, prompt, max_new, spec_k=5, eos=(151645, 151643)):
    prompt = np.ascontiguousarray(prompt, np.uint32)
    eos_a = np.asarray(eos, np.uint32)
    out = np.empty(max_new + spec_k, np.uint32)
    n = INT()
    stats = np.zeros(3, np.int64)
    _chk(lib().orc_speculative_generate(target.h, tcache.h, draft.h, dcache.h, _p(prompt), prompt.size, max_new,
                                        spec_k, _p(eos_a), eos_a.size, _p(out), ctypes.byref(n), _p(stats)))
    return out[: n.value], stats
