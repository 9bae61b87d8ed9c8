"""Pins the oracle's ops around the matmul against library routines (torch
float64, numpy) and closed forms: RMSNorm (qwen3.rs:44-55), rotate-half
RoPE (qwen3.rs:407-413), slice_update (mlx_ext.rs:21-64), GQA SDPA with
the causal-offset mask (qwen3.rs:491-518, 629-653), SwiGLU
(kernels.rs:73-74) and argmax (engine.rs:195-202)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _util import bf16_to_f32, max_rel_err


def bf16_of(a, orc):
    return orc.f32_to_bf16(np.asarray(a, np.float32))


def test_rms_norm_closed_form_and_torch(orc):
    # constant rows: x / rms(x) = sign(x) exactly (up to eps)
    x = bf16_of(np.array([[3.0] * 64, [-0.5] * 64]), orc)
    w = bf16_of(np.linspace(0.5, 2.0, 64), orc)
    y = bf16_to_f32(orc.rms_norm(x, w))
    np.testing.assert_allclose(y[0], bf16_to_f32(w), rtol=2 ** -7)
    np.testing.assert_allclose(y[1], -bf16_to_f32(w), rtol=2 ** -7)
    rng = np.random.default_rng(0)
    x = bf16_of(rng.standard_normal((33, 2560)) * 3, orc)
    w = bf16_of(rng.uniform(0.5, 1.5, 2560), orc)
    ref = F.rms_norm(torch.from_numpy(bf16_to_f32(x)).double(), (2560,), torch.from_numpy(bf16_to_f32(w)).double(),
                     eps=1e-6).numpy()
    y = bf16_to_f32(orc.rms_norm(x, w, 1e-6))
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-3)) < 2 ** -6


def test_rope_identity_norm_and_complex_rotation(orc):
    rng = np.random.default_rng(1)
    H, T, D, theta = 4, 7, 128, 1e6
    x = bf16_of(rng.standard_normal((H, T, D)), orc)
    # position 0 -> identity (bit exact)
    y0 = orc.rope(x[:, :1], theta, 0)
    np.testing.assert_array_equal(y0, x[:, :1])
    # against complex multiplication z * exp(i p f) in float64
    off = 4090
    y = bf16_to_f32(orc.rope(x, theta, off)).astype(np.float64)
    xf = bf16_to_f32(x).astype(np.float64)
    half = D // 2
    f = theta ** (-np.arange(half) / half)
    ang = (off + np.arange(T))[:, None] * f[None, :]
    z = (xf[..., :half] + 1j * xf[..., half:]) * np.exp(1j * ang)[None]
    ref = np.concatenate([z.real, z.imag], -1)
    assert np.max(np.abs(y - ref)) < 2e-2 * np.max(np.abs(ref))
    # each rotated pair keeps its norm
    n_in = np.hypot(xf[..., :half], xf[..., half:])
    n_out = np.hypot(y[..., :half], y[..., half:])
    np.testing.assert_allclose(n_out, n_in, rtol=1e-2, atol=1e-2)


def test_rope_relative_position(orc):
    """<rope(q, m), rope(k, n)> depends only on m - n."""
    rng = np.random.default_rng(2)
    q = bf16_of(rng.standard_normal((1, 1, 128)), orc)
    k = bf16_of(rng.standard_normal((1, 1, 128)), orc)
    dots = []
    for m, n in [(10, 3), (107, 100), (1007, 1000)]:
        a = bf16_to_f32(orc.rope(q, 1e6, m)).astype(np.float64).ravel()
        b = bf16_to_f32(orc.rope(k, 1e6, n)).astype(np.float64).ravel()
        dots.append(a @ b)
    assert np.ptp(dots) < 0.05 * abs(dots[0]) + 0.05


def test_slice_update_numpy_semantics(orc):
    rng = np.random.default_rng(3)
    src = rng.integers(0, 60000, (8, 64, 128)).astype(np.uint16)
    ref = src.copy()
    upd = rng.integers(0, 60000, (8, 5, 128)).astype(np.uint16)
    assert orc.slice_update(src, upd, [0, 59, 0], [8, 64, 128], [1, 1, 1]) == 0
    ref[0:8, 59:64, 0:128] = upd
    np.testing.assert_array_equal(src, ref)
    upd2 = rng.integers(0, 60000, (4, 3, 32)).astype(np.uint16)
    assert orc.slice_update(src, upd2, [1, 2, 0], [8, 9, 128], [2, 3, 4]) == 0
    ref[1:8:2, 2:9:3, 0:128:4] = upd2
    np.testing.assert_array_equal(src, ref)
    # out-of-range stop is an error and writes nothing
    before = src.copy()
    assert orc.slice_update(src, upd, [0, 60, 0], [8, 65, 128], [1, 1, 1]) != 0
    np.testing.assert_array_equal(src, before)


def _sdpa_torch(q, k, v, L, offset, causal, scale):
    Hq, M, D = q.shape
    Hkv = k.shape[0]
    qt = torch.from_numpy(bf16_to_f32(q)).double()[None]
    kt = torch.from_numpy(bf16_to_f32(k[:, :L])).double().repeat_interleave(Hq // Hkv, 0)[None]
    vt = torch.from_numpy(bf16_to_f32(v[:, :L])).double().repeat_interleave(Hq // Hkv, 0)[None]
    mask = None
    if causal:
        mask = torch.tril(torch.ones(M, L, dtype=torch.bool), diagonal=offset)
    out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return out[0].transpose(0, 1).reshape(M, Hq * D).numpy()


@pytest.mark.parametrize("Hq,Hkv,M,offset", [(4, 2, 1, 37), (8, 2, 5, 90), (4, 4, 9, 0), (32, 8, 1, 300)])
def test_sdpa_vs_torch(orc, Hq, Hkv, M, offset):
    rng = np.random.default_rng(Hq * 100 + M)
    D, cap = 128, offset + M + 3
    q = bf16_of(rng.standard_normal((Hq, M, D)), orc)
    k = bf16_of(rng.standard_normal((Hkv, cap, D)), orc)
    v = bf16_of(rng.standard_normal((Hkv, cap, D)), orc)
    L = offset + M
    scale = 1 / np.sqrt(D)
    y = bf16_to_f32(orc.sdpa(q, k, v, L, offset, M > 1, scale))
    ref = _sdpa_torch(q, k, v, L, offset, M > 1, scale)
    assert max_rel_err(y, ref) < 1e-2


def test_sdpa_closed_forms(orc):
    rng = np.random.default_rng(5)
    D = 128
    q = bf16_of(rng.standard_normal((2, 1, D)), orc)
    v = bf16_of(rng.standard_normal((1, 4, D)), orc)
    # one key -> output is that value row
    k = bf16_of(rng.standard_normal((1, 4, D)), orc)
    y = orc.sdpa(q, k, v, 1, 0, False, 0.1)
    np.testing.assert_array_equal(y.reshape(2, D), np.stack([v[0, 0], v[0, 0]]))
    # identical keys -> mean of the values
    k_eq = np.repeat(k[:, :1], 4, axis=1)
    y = bf16_to_f32(orc.sdpa(q, k_eq, v, 4, 0, False, 0.1)).reshape(2, D)
    mean = bf16_to_f32(v[0]).mean(0)
    np.testing.assert_allclose(y[0], mean, rtol=1e-2, atol=1e-2)


def test_silu_mul_vs_torch(orc):
    rng = np.random.default_rng(6)
    g = bf16_of(rng.standard_normal(4096) * 4, orc)
    u = bf16_of(rng.standard_normal(4096), orc)
    y = bf16_to_f32(orc.silu_mul(g, u))
    ref = (F.silu(torch.from_numpy(bf16_to_f32(g)).double()) * torch.from_numpy(bf16_to_f32(u)).double()).numpy()
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-2)) < 2 ** -6


def test_argmax_first_index_on_ties(orc):
    rng = np.random.default_rng(7)
    x = bf16_of(rng.standard_normal((5, 151936)), orc)
    x[1, 100] = x[1, 5000] = bf16_of([50.0], orc)[0]
    x[2, :] = bf16_of([1.0], orc)[0]
    got = orc.argmax_rows(x)
    ref = np.argmax(bf16_to_f32(x), axis=1)  # numpy: first index of the max
    np.testing.assert_array_equal(got, ref)
    assert got[1] == 100 and got[2] == 0


def test_reversed_accumulation_sdpa_and_rms_norm(orc):
    """Reversed key and square orders: closed forms stay exact (one visible
    key returns v; constant rows normalise to the weight), random inputs
    move by rounding only."""
    rng = np.random.default_rng(5)
    Hq, Hkv, D, L = 8, 2, 128, 300
    q = bf16_of(rng.standard_normal((Hq, 1, D)), orc)
    k = bf16_of(rng.standard_normal((Hkv, L, D)), orc)
    v = bf16_of(rng.standard_normal((Hkv, L, D)), orc)
    scale = 1.0 / np.sqrt(D)
    with orc.reversed_accumulation():
        one = orc.sdpa(q, k, v, 1, 0, False, scale)
        rev = orc.sdpa(q, k, v, L, 0, False, scale)
    np.testing.assert_array_equal(one.reshape(Hq, D), np.repeat(v[:, 0], Hq // Hkv, axis=0))
    fwd = orc.sdpa(q, k, v, L, 0, False, scale)
    f, r = bf16_to_f32(fwd), bf16_to_f32(rev)
    assert np.any(f != r)
    assert np.max(np.abs(f - r)) <= 4 * 2.0 ** -8 * np.max(np.abs(f))
    x = bf16_of(np.array([[3.0] * 256]), orc)
    w = bf16_of(np.linspace(0.5, 2.0, 256), orc)
    with orc.reversed_accumulation():
        yc = orc.rms_norm(x, w)
    np.testing.assert_array_equal(yc, orc.rms_norm(x, w))
    x = bf16_of(rng.standard_normal((16, 2560)) * 3, orc)
    w = bf16_of(rng.uniform(0.5, 1.5, 2560), orc)
    fwd = bf16_to_f32(orc.rms_norm(x, w))
    with orc.reversed_accumulation():
        rev = bf16_to_f32(orc.rms_norm(x, w))
    assert np.max(np.abs(fwd - rev) / np.maximum(np.abs(fwd), 1e-3)) <= 2 * 2.0 ** -8
