"""Writes the golden fixtures of tests/golden/ from closed forms (numpy only;
no oracle, no GPU).  Run from the repository root:

    python tests/golden/make_golden.py

Fixtures (all inputs seeded, all expected outputs computed in float64 and
rounded to bf16 with round-to-nearest-even where the op returns bf16):
  dyadic_qmm.npz   quantized matmul with dyadic x, s, b (M = 1, 3, 8, 1, 12): every product and
                   partial sum is exact in fp32, so y is exact; also the
                   dequantized weights (exact in bf16)
  pack_table.npz   u32 words and their 8 nibbles, element j at bits 4j..4j+3
  tiny_qmm_f64.npz random small shapes, y in float64
  rope.npz         rotate-half RoPE (theta 1e6) at offsets 0, 1, 4095
  kv_write.npz     slice_update of [8, M=3, 128] rows at offset cap - M
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f64_to_bf16_exact(v):
    """float64 -> bf16 RNE without an intermediate float32 rounding."""
    v = np.asarray(v, np.float64)
    out = np.zeros(v.shape, np.uint16)
    flat, res = v.ravel(), out.ravel()
    for i, x in enumerate(flat):
        if x == 0.0:
            res[i] = 0x8000 if np.signbit(x) else 0
            continue
        m, e = np.frexp(abs(x))            # x = m * 2^e, m in [0.5, 1)
        q = np.round(m * 256.0)             # 8 significant bits, ties to even
        if q == 256.0:
            q, e = 128.0, e + 1
        val = np.float32(q / 256.0 * 2.0 ** e)
        bits = int(np.array(val, np.float32).view(np.uint32)) >> 16
        res[i] = bits | (0x8000 if x < 0 else 0)
    return out


def bf16_to_f64(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def pack(q):
    """q [N, K] in 0..15 -> [N, K/8] u32, element j of a word at bits 4j."""
    N, K = q.shape
    q = q.reshape(N, K // 8, 8).astype(np.uint32)
    return np.bitwise_or.reduce(q << (4 * np.arange(8, dtype=np.uint32)), axis=2).astype(np.uint32)


def dyadic(rng, M, N, K):
    G = K // 64
    q = rng.integers(0, 16, (N, K))
    s = 2.0 ** rng.integers(-4, 0, (N, G))            # 1/16 .. 1/2
    b = rng.integers(-16, 17, (N, G)) / 8.0           # multiples of 1/8 in [-2, 2]
    x = rng.choice([-2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0], (M, K))
    deq = s.repeat(64, 1) * q + b.repeat(64, 1)       # exact (<= 7 significant bits)
    y = x @ deq.T                                     # exact: multiples of 1/16 below 2^15
    return dict(x=f64_to_bf16_exact(x), w=pack(q), s=f64_to_bf16_exact(s), b=f64_to_bf16_exact(b),
                deq=f64_to_bf16_exact(deq), y=f64_to_bf16_exact(y), y64=y)


def main():
    rng = np.random.default_rng(20260101)
    d = {}
    for i, (M, N, K) in enumerate([(1, 16, 128), (3, 37, 192), (8, 64, 512), (1, 24, 2560), (12, 64, 512)]):
        for k, v in dyadic(rng, M, N, K).items():
            d[f"{k}_{i}"] = v
    np.savez_compressed(os.path.join(HERE, "dyadic_qmm.npz"), **d)

    words = rng.integers(0, 2 ** 32, 256, dtype=np.uint64).astype(np.uint32)
    words[:4] = [0x00000000, 0xFFFFFFFF, 0x76543210, 0xFEDCBA98]
    nib = ((words[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).astype(np.uint8)
    np.savez_compressed(os.path.join(HERE, "pack_table.npz"), words=words, nibbles=nib)

    t = {}
    for i, (M, N, K) in enumerate([(1, 64, 256), (5, 33, 128), (2, 96, 1024)]):
        G = K // 64
        q = rng.integers(0, 16, (N, K))
        s = f64_to_bf16_exact(rng.uniform(0.002, 0.02, (N, G)))
        b = f64_to_bf16_exact(-8.0 * bf16_to_f64(s) + rng.normal(0, 0.002, (N, G)))
        x = f64_to_bf16_exact(rng.normal(0, 1, (M, K)))
        deq = bf16_to_f64(s).repeat(64, 1) * q + bf16_to_f64(b).repeat(64, 1)
        t.update({f"x_{i}": x, f"w_{i}": pack(q), f"s_{i}": s, f"b_{i}": b, f"y64_{i}": bf16_to_f64(x) @ deq.T})
    np.savez_compressed(os.path.join(HERE, "tiny_qmm_f64.npz"), **t)

    x = f64_to_bf16_exact(rng.normal(0, 1, (2, 3, 128)))
    r = {"x": x}
    xf = bf16_to_f64(x)
    inv = 1e6 ** (-np.arange(64) * 2.0 / 128.0)
    for off in (0, 1, 4095):
        ang = (off + np.arange(3))[:, None] * inv[None, :]          # [T, 64]
        c, sn = np.cos(ang), np.sin(ang)
        a, bb = xf[..., :64], xf[..., 64:]
        r[f"y_{off}"] = f64_to_bf16_exact(np.concatenate([a * c - bb * sn, a * sn + bb * c], -1))
    np.savez_compressed(os.path.join(HERE, "rope.npz"), **r)

    cap, M = 16, 3
    src = f64_to_bf16_exact(rng.normal(0, 1, (8, cap, 128)))
    upd = f64_to_bf16_exact(rng.normal(0, 1, (8, M, 128)))
    after = src.copy()
    after[:, cap - M:cap, :] = upd
    np.savez_compressed(os.path.join(HERE, "kv_write.npz"), src=src, update=upd, after=after,
                        start=np.array([0, cap - M, 0]), stop=np.array([8, cap, 128]), strides=np.array([1, 1, 1]))


if __name__ == "__main__":
    main()
