"""Pins the CPU oracle's MLX-format arithmetic against known answers,
closed forms and library routines (numpy / torch), independently of the
oracle's own loops.

Covers the format rows: pack/unpack order, dequantize (qwen3.rs:69-76),
quantized_matmul (qwen3.rs:30-41), the quantizer used for random init and
the seeded generator.
"""
import numpy as np
import pytest
import torch

from _util import bf16_to_f32, max_rel_err


def test_bf16_rounding_matches_torch(orc):
    rng = np.random.default_rng(0)
    f = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -0.0, np.inf, -np.inf, 3.3895e38], np.float32),
    ]).astype(np.float32)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.f32_to_bf16(f)
    np.testing.assert_array_equal(got, ref)
    # single-value C path agrees with the vectorised one
    for v in f[-7:]:
        assert orc.lib().orc_f2bf(float(v)) == orc.f32_to_bf16(np.array([v], np.float32))[0]


def test_generator_moments_and_determinism(orc):
    a = orc.fill_normal_f32(1234, 1 << 20, sigma=0.02)
    b = orc.fill_normal_f32(1234, 1 << 20, sigma=0.02)
    np.testing.assert_array_equal(a, b)
    assert abs(a.mean()) < 1e-4
    assert abs(a.std() - 0.02) / 0.02 < 2e-3
    # Irwin-Hall(4) kurtosis is 3 - 6/(5*4) = 2.7
    k = np.mean((a / a.std()) ** 4)
    assert abs(k - 2.7) < 0.02
    # bf16 fill is the RNE rounding of the same deviates
    h = orc.fill_normal_bf16(1234, 4096, sigma=0.02)
    np.testing.assert_array_equal(h, orc.f32_to_bf16(a[:4096]))
    c = orc.fill_normal_f32(1235, 4096, sigma=0.02)
    assert not np.array_equal(a[:4096], c)


def test_pack_order_known_answer(orc):
    # A group whose values sit exactly on the 16-level grid of
    # s = 2^-4, beta = -0.5 quantizes to known nibbles; element k of a row
    # lives in word k//8 at bits 4*(k%8) (lowest nibble first).
    q = np.array([(k * 7 + 3) % 16 for k in range(64)], np.int64)
    q[5], q[9] = 0, 15  # make min / max exactly beta and beta + 15 s
    w = (-0.5 + q * 2.0 ** -4).astype(np.float32)[None, :]
    wq, s, b = orc.quantize(w)
    assert bf16_to_f32(s)[0, 0] == 2.0 ** -4
    assert bf16_to_f32(b)[0, 0] == -0.5
    # hand-derived: q[0:8] = 3,A,1,8,F,0,D,4 and q[8:16] = B,F,9,0,7,E,5,C
    assert int(wq[0, 0]) == 0x4D0F81A3
    assert int(wq[0, 1]) == 0xC5E709FB


def test_dequant_dyadic_exact(orc):
    # dyadic scales/biases: every s*q+b is exact in bf16 -> bit-exact
    rng = np.random.default_rng(1)
    N, K = 16, 256
    wq = rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = orc.f32_to_bf16((2.0 ** rng.integers(-8, -2, (N, K // 64))).astype(np.float32))
    b = orc.f32_to_bf16((-(2.0 ** rng.integers(-3, 1, (N, K // 64)))).astype(np.float32))
    out = bf16_to_f32(orc.dequantize(wq, s, b))
    nib = (wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    q = nib.reshape(N, K).astype(np.float64)
    ref = np.repeat(bf16_to_f32(s), 64, axis=1) * q + np.repeat(bf16_to_f32(b), 64, axis=1)
    np.testing.assert_array_equal(out.astype(np.float64), ref)


def test_dequant_general_matches_torch_rounding(orc):
    wq, s, b = orc.init_qlinear(77, 64, 512)
    out = orc.dequantize(wq, s, b)
    nib = (wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    q = torch.from_numpy(nib.reshape(64, 512).astype(np.float32))
    sf = torch.from_numpy(np.repeat(bf16_to_f32(s), 64, axis=1))
    bf = torch.from_numpy(np.repeat(bf16_to_f32(b), 64, axis=1))
    ref = (sf * q + bf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(out, ref)
    # gather = dequantize of the selected rows
    ids = np.array([5, 0, 63, 5], np.uint32)
    np.testing.assert_array_equal(orc.dequant_gather(ids, wq, s, b), out[ids])


def test_quantizer_reconstruction_bound(orc):
    w = orc.fill_normal_f32(9, 32 * 1024, sigma=0.02).reshape(32, 1024)
    wq, s, b = orc.quantize(w)
    deq = bf16_to_f32(orc.dequantize(wq, s, b)).astype(np.float64)
    step = np.repeat(bf16_to_f32(s).astype(np.float64), 64, axis=1)
    # |w - s*q - b| <= s/2 plus the bf16 rounding of s, b and the output
    err = np.abs(deq - w)
    assert np.all(err <= 0.5 * step * 1.02 + np.abs(w) * 2 ** -8 + 2 ** -8 * step * 16)
    # group min maps to q = 0 and group max to q = 15
    nib = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(32, 1024)
    g = nib.reshape(32, 16, 64)
    wg = w.reshape(32, 16, 64)
    assert np.all(np.take_along_axis(g, wg.argmin(-1)[..., None], -1) == 0)
    assert np.all(np.take_along_axis(g, wg.argmax(-1)[..., None], -1) == 15)


def test_init_qlinear_is_exact_affine_quantization(orc):
    """init_qlinear evaluates the affine formula exactly on the integer
    deviates: it agrees with the float quantizer of the same deviates except
    where float rounding of (w - min) / s lands on a .5 boundary."""
    N, K = 64, 1024
    w = orc.fill_normal_f32(9, N * K, sigma=0.02).reshape(N, K)
    wq_f, s_f, b_f = orc.quantize(w)
    wq, s, b = orc.init_qlinear(9, N, K)
    np.testing.assert_array_equal(b, b_f)  # group minimum
    assert np.max(np.abs(bf16_to_f32(s) - bf16_to_f32(s_f)) / bf16_to_f32(s_f)) <= 2 ** -8
    nib = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K)
    nib_f = ((wq_f[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K)
    assert np.mean(nib == nib_f) > 0.999
    assert np.max(np.abs(nib.astype(int) - nib_f)) <= 1
    # exact integer reference: t recovered from the float deviates (t * c)
    t = np.rint(w.astype(np.float64) / np.float64(orc.sigma_to_c(0.02))).astype(np.int64).reshape(N, K // 64, 64)
    lo, hi = t.min(-1, keepdims=True), t.max(-1, keepdims=True)
    num, den = 15 * (t - lo), hi - lo
    q = num // den
    r = num - q * den
    q += (2 * r > den) | ((2 * r == den) & (q % 2 == 1))
    np.testing.assert_array_equal(nib.reshape(N, K // 64, 64), q)


def _pack(q):
    N, K = q.shape
    q = q.reshape(N, K // 8, 8).astype(np.uint32)
    return np.bitwise_or.reduce(q << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)


@pytest.mark.parametrize("M,N,K", [(1, 37, 64), (3, 64, 512), (8, 128, 1024)])
def test_qmatmul_integer_exact(orc, M, N, K):
    # s = 1, b = 1, x in {-1, 0, 1}: y = sum (q+1) x is a small integer, exact
    rng = np.random.default_rng(M * 1000 + N)
    q = rng.integers(0, 16, (N, K))
    wq = _pack(q)
    s = np.full((N, K // 64), 0x3F80, np.uint16)
    b = np.full((N, K // 64), 0x3F80, np.uint16)
    xi = rng.integers(-1, 2, (M, K))
    for m in range(M):  # a nonzero row sum makes the bias term visible
        if xi[m].sum() == 0:
            xi[m, np.flatnonzero(xi[m] == 0)[0]] = 1
    x = orc.f32_to_bf16(xi.astype(np.float32))
    y = bf16_to_f32(orc.qmatmul(x, wq, s, b))
    ref = xi @ (q + 1).T  # |ref| < 256 -> exact in bf16 when |ref| <= 256
    small = np.abs(ref) <= 256
    assert small.mean() > 0.5
    np.testing.assert_array_equal(y[small], ref[small].astype(np.float32))
    # a dropped bias term or a transposed / reordered unpack would not survive
    assert not np.any(y[small] == (xi @ q.T)[small])
    q_rev = q.reshape(N, K // 8, 8)[:, :, ::-1].reshape(N, K)
    assert not np.array_equal(y[small], (xi @ (q_rev + 1).T)[small].astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(1, 256, 2560), (5, 96, 4096), (16, 64, 9728)])
def test_qmatmul_vs_float64_matmul(orc, M, N, K):
    wq, s, b = orc.init_qlinear(100 + M, N, K)
    x = orc.fill_normal_bf16(200 + M, M * K).reshape(M, K)
    y = bf16_to_f32(orc.qmatmul(x, wq, s, b))
    nib = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K)
    Wx = np.repeat(bf16_to_f32(s), 64, 1).astype(np.float64) * nib + np.repeat(bf16_to_f32(b), 64, 1)
    ref = bf16_to_f32(x).astype(np.float64) @ Wx.T  # numpy BLAS, float64
    assert max_rel_err(y, ref) < 1e-2
    # per element: bf16 output rounding (2^-9 rel) plus fp32 accumulation error
    tol = np.abs(ref) * 2 ** -8 + 1e-5 * np.sqrt(K) * np.max(np.abs(ref))
    assert np.all(np.abs(y - ref) <= tol)
    # the float64 yardstick of the oracle agrees with numpy
    np.testing.assert_allclose(orc.qmatmul_f64(x, wq, s, b), ref, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("M,N,K", [(9, 64, 512), (16, 96, 2560), (37, 40, 4096)])
def test_qmm_dequant_vs_float64_on_dequantized_weights(orc, M, N, K):
    """Matrix path: y = bf16(x w^T) with w the bf16 weights orc.dequantize
    returns (pinned bit-exact separately); numpy float64 on those same bf16
    weights is the yardstick, so a dropped scale / bias, a transposed operand
    or a skipped weight rounding shows up well above the fp32 summation bar."""
    wq, s, b = orc.init_qlinear(300 + M, N, K)
    x = orc.fill_normal_bf16(400 + M, M * K).reshape(M, K)
    y = bf16_to_f32(orc.qmm_dequant(x, wq, s, b))
    w16 = bf16_to_f32(orc.dequantize(wq, s, b)).astype(np.float64)
    ref = bf16_to_f32(x).astype(np.float64) @ w16.T
    # bf16 output rounding (2^-9 relative) plus fp32 accumulation error
    tol = np.abs(ref) * 2 ** -8 + 1e-5 * np.sqrt(K) * np.max(np.abs(ref))
    assert np.all(np.abs(y - ref) <= tol)
    # the unrounded weights (s*q + b in float64) give a measurably different
    # product: the weight rounding is really there
    nib = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K)
    wx = np.repeat(bf16_to_f32(s), 64, 1).astype(np.float64) * nib + np.repeat(bf16_to_f32(b), 64, 1)
    assert np.max(np.abs(w16 - wx)) > 0
    # dispatch: qlinear is qmatmul up to 8 rows and qmm_dequant beyond
    np.testing.assert_array_equal(orc.qlinear(x, wq, s, b), orc.qmm_dequant(x, wq, s, b))
    np.testing.assert_array_equal(orc.qlinear(x[:8], wq, s, b), orc.qmatmul(x[:8], wq, s, b))


@pytest.mark.parametrize("M,x_bcast", [(1, 4), (3, 1)])
def test_gather_qmm_vs_float64(orc, M, x_bcast):
    """Routed qmm: route r is x block r // x_bcast times expert rhs[r]; numpy
    float64 on the exact dequantized experts is the yardstick.  A route
    reading the wrong expert or the wrong x block (r % blocks instead of
    r // x_bcast) fails the per-element bound."""
    E, N, K, R = 5, 40, 256, 8
    ex = [orc.init_qlinear(700 + e, N, K) for e in range(E)]
    wq = np.stack([t[0] for t in ex])
    s = np.stack([t[1] for t in ex])
    b = np.stack([t[2] for t in ex])
    rhs = np.array([3, 0, 3, 4, 1, 1, 2, 0], np.uint32)
    blocks = R // x_bcast
    x = orc.fill_normal_bf16(800 + M, blocks * M * K).reshape(blocks, M, K)
    y = bf16_to_f32(orc.gather_qmm(x, wq, s, b, rhs, x_bcast))
    nib = ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(E, N, K)
    Wx = np.repeat(bf16_to_f32(s), 64, 2).astype(np.float64) * nib + np.repeat(bf16_to_f32(b), 64, 2)
    xf = bf16_to_f32(x).astype(np.float64)

    def ref_for(block_of):
        return np.stack([xf[block_of(r)] @ Wx[rhs[r]].T for r in range(R)])

    ref = ref_for(lambda r: r // x_bcast)
    tol = np.abs(ref) * 2 ** -8 + 1e-5 * np.sqrt(K) * np.max(np.abs(ref))
    assert np.all(np.abs(y - ref) <= tol)
    if x_bcast > 1:
        wrong = ref_for(lambda r: r % blocks)
        assert not np.all(np.abs(y - wrong) <= tol)
    # each route is exactly quantized_matmul on its expert
    r = 2
    np.testing.assert_array_equal(orc.gather_qmm(x, wq, s, b, rhs, x_bcast)[r],
                                  orc.qmatmul(x[r // x_bcast], wq[rhs[r]], s[rhs[r]], b[rhs[r]]))
    # ids past the last expert are clamped to it
    hi = rhs.copy()
    hi[5] = 77
    clamp = rhs.copy()
    clamp[5] = E - 1
    np.testing.assert_array_equal(orc.gather_qmm(x, wq, s, b, hi, x_bcast), orc.gather_qmm(x, wq, s, b, clamp, x_bcast))


@pytest.mark.parametrize("M,N,K", [(1, 8192, 2560), (5, 2048, 4096), (12, 1024, 1024)])
def test_reversed_accumulation_is_a_pure_reordering(orc, M, N, K):
    """The reordered oracle (the summation-order floor of the end-to-end
    bar) must change nothing but the order of fp32 additions: on sums that
    are exact in fp32 it gives the forward bits, on random data it differs
    from the forward order somewhere (it is on) but only by rounding, and it
    switches off again on leaving the context.  (Enough outputs that some
    bf16 rounding flips with the order.)"""
    rng = np.random.default_rng(M * 7 + K)
    # exact sums: s = 1, b = 1, x in {-1, 0, 1}
    q = rng.integers(0, 16, (N, K))
    wq = _pack(q)
    one = np.full((N, K // 64), 0x3F80, np.uint16)
    xi = orc.f32_to_bf16(rng.integers(-1, 2, (M, K)).astype(np.float32))
    fwd = orc.qlinear(xi, wq, one, one)
    with orc.reversed_accumulation():
        rev = orc.qlinear(xi, wq, one, one)
    np.testing.assert_array_equal(rev, fwd)
    # random data: rounding-level differences only
    wq, s, b = orc.init_qlinear(300 + M, N, K)
    x = orc.fill_normal_bf16(400 + M, M * K).reshape(M, K)
    fwd = orc.qlinear(x, wq, s, b)
    with orc.reversed_accumulation():
        rev = orc.qlinear(x, wq, s, b)
    after = orc.qlinear(x, wq, s, b)
    np.testing.assert_array_equal(after, fwd)
    f, r = bf16_to_f32(fwd), bf16_to_f32(rev)
    ref = orc.qmatmul_f64(x, wq, s, b)
    assert np.any(f != r)
    assert np.max(np.abs(f - r)) <= 2 * 2.0 ** -7 * np.max(np.abs(ref))
    assert np.max(np.abs(r - ref)) / np.max(np.abs(ref)) < 1e-2
