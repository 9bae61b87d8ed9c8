"""GPU parity of the ops around the matmul and of the MFMA qmm against the
CPU oracle on identical inputs (bf16 out; tolerances in each test)."""
import numpy as np
import pytest

from _util import bf16_to_f32, bf16_ulp_diff, max_rel_err, to_torch_bf16, torch_bf16_bits, u32_of

pytestmark = pytest.mark.gpu


def _close(y_bits, ref_bits, ulps=2, floor=1e-3):
    y = bf16_to_f32(y_bits).astype(np.float64)
    r = bf16_to_f32(ref_bits).astype(np.float64)
    ok = np.abs(y - r) <= np.maximum(ulps * np.abs(r) * 2.0 ** -7, floor * np.max(np.abs(r)))
    return ok.mean()


def test_rms_norm(gpu, orc):
    x = gpu.fill_normal_bf16(1, (37, 2560), sigma=2.0)
    w = gpu.fill_normal_bf16(2, (2560,), sigma=0.5)
    y = gpu.rms_norm(x, w, 1e-6)
    ref = orc.rms_norm(torch_bf16_bits(x), torch_bf16_bits(w), 1e-6)
    assert _close(torch_bf16_bits(y), ref) == 1.0


@pytest.mark.parametrize("offset", [0, 1, 4095])
def test_rope(gpu, orc, offset):
    x = gpu.fill_normal_bf16(3, (8, 5, 128))
    y = gpu.rope(x, 1e6, offset)
    ref = orc.rope(torch_bf16_bits(x), 1e6, offset)
    assert _close(torch_bf16_bits(y), ref) == 1.0


def test_slice_update(gpu, orc):
    import torch

    src = gpu.fill_normal_bf16(4, (8, 64, 128))
    upd = gpu.fill_normal_bf16(5, (4, 3, 32))
    ref = torch_bf16_bits(src).copy()
    gpu.slice_update(src, upd, [1, 2, 0], [8, 9, 128], [2, 3, 4])
    ref[1:8:2, 2:9:3, 0:128:4] = torch_bf16_bits(upd)
    np.testing.assert_array_equal(torch_bf16_bits(src), ref)
    with pytest.raises(gpu.BmxError):
        gpu.slice_update(src, upd, [1, 2, 0], [8, 9, 129], [2, 3, 4])
    torch.cuda.synchronize()


# (the kernel takes heads in groups of 8: 12 / 4 and 20 / 10 leave partial groups)
@pytest.mark.parametrize("M,offset,Hq,Hkv", [(1, 0, 32, 8), (1, 100, 32, 8), (5, 60, 32, 8), (20, 0, 32, 8),
                                             (20, 13, 32, 8), (20, 13, 12, 4), (3, 5, 20, 10)])
def test_qk_norm_rope_kv(gpu, orc, M, offset, Hq, Hkv):
    import torch

    cap = 128
    q = gpu.fill_normal_bf16(6, (M, Hq * 128), sigma=3.0)
    k = gpu.fill_normal_bf16(7, (M, Hkv * 128), sigma=3.0)
    v = gpu.fill_normal_bf16(8, (M, Hkv * 128))
    qn = gpu.fill_normal_bf16(9, (128,), sigma=0.3)
    kn = gpu.fill_normal_bf16(10, (128,), sigma=0.3)
    kc = torch.zeros(Hkv, cap, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    qo = gpu.qk_norm_rope_kv(q, k, v, qn, kn, kc, vc, offset, 1e-6, 1e6)
    torch.cuda.synchronize()
    # oracle: per-head norm, [H, M, 128] transpose, rope, slice write
    qb = orc.rms_norm(torch_bf16_bits(q).reshape(M * Hq, 128), torch_bf16_bits(qn)).reshape(M, Hq, 128)
    kb = orc.rms_norm(torch_bf16_bits(k).reshape(M * Hkv, 128), torch_bf16_bits(kn)).reshape(M, Hkv, 128)
    qr = orc.rope(np.ascontiguousarray(qb.transpose(1, 0, 2)), 1e6, offset)
    kr = orc.rope(np.ascontiguousarray(kb.transpose(1, 0, 2)), 1e6, offset)
    assert _close(torch_bf16_bits(qo), qr) == 1.0
    kcg, vcg = torch_bf16_bits(kc), torch_bf16_bits(vc)
    assert _close(kcg[:, offset:offset + M], kr) == 1.0
    np.testing.assert_array_equal(vcg[:, offset:offset + M], torch_bf16_bits(v).reshape(M, Hkv, 128).transpose(1, 0, 2))
    # nothing outside the written rows
    assert not kcg[:, :offset].any() and not kcg[:, offset + M:].any()
    with pytest.raises(gpu.BmxError) as ei:
        gpu.qk_norm_rope_kv(q, k, v, qn, kn, kc, vc, cap - M + 1)
    assert ei.value.code == gpu.BMX_E_KV_CAPACITY


@pytest.mark.parametrize("Hq,Hkv,M,offset", [(32, 8, 1, 0), (32, 8, 1, 4095), (32, 8, 1, 777), (16, 8, 1, 31),
                                             (32, 8, 5, 2043), (64, 8, 5, 300), (32, 8, 3, 100), (64, 8, 8, 1000),
                                             (32, 8, 37, 0), (32, 8, 40, 100), (32, 8, 200, 0), (16, 8, 130, 70),
                                             (32, 8, 513, 3), (8, 8, 100, 0), (24, 8, 90, 3), (64, 8, 300, 17)])
def test_attention(gpu, orc, Hq, Hkv, M, offset):
    cap = offset + M + 5
    q = gpu.fill_normal_bf16(11, (Hq, M, 128))
    kc = gpu.fill_normal_bf16(12, (Hkv, cap, 128))
    vc = gpu.fill_normal_bf16(13, (Hkv, cap, 128))
    scale = 1 / np.sqrt(128)
    ref = orc.sdpa(torch_bf16_bits(q), torch_bf16_bits(kc), torch_bf16_bits(vc), offset + M, offset, M > 1,
                   np.float32(scale))
    for ws in (True, False):
        y = gpu.attention(q, kc, vc, offset, scale, use_workspace=ws)
        yb = torch_bf16_bits(y)
        assert max_rel_err(bf16_to_f32(yb), bf16_to_f32(ref)) < 1e-2
        assert _close(yb, ref, ulps=2, floor=2e-3) > 0.999


@pytest.mark.parametrize("M,offset", [(130, 70), (300, 0)])
def test_attention_prefill_v_beyond_fp16_range(gpu, orc, M, offset):
    """The prefill kernel multiplies p by an fp16 copy of V; a key block with
    a V value beyond fp16's range (here keys 64..127 scaled by 2^17, about
    1.3e5) must take the two-term bf16 product instead, or those keys'
    contributions would saturate at 65504."""
    Hq, Hkv = 32, 8
    cap = offset + M + 5
    q = gpu.fill_normal_bf16(21, (Hq, M, 128))
    kc = gpu.fill_normal_bf16(22, (Hkv, cap, 128))
    vc = gpu.fill_normal_bf16(23, (Hkv, cap, 128))
    vc[:, 64:128] *= 2.0 ** 17  # exact in bf16
    assert float(vc.float().abs().max()) > 65504.0
    scale = 1 / np.sqrt(128)
    ref = orc.sdpa(torch_bf16_bits(q), torch_bf16_bits(kc), torch_bf16_bits(vc), offset + M, offset, True,
                   np.float32(scale))
    yb = torch_bf16_bits(gpu.attention(q, kc, vc, offset, scale))
    assert max_rel_err(bf16_to_f32(yb), bf16_to_f32(ref)) < 1e-2
    assert _close(yb, ref, ulps=2, floor=2e-3) > 0.999


def test_attention_workspace_reuse(gpu, orc):
    """One zero-filled workspace over calls of different split counts and row
    tilings: the arrival counters come back to zero after every call."""
    import torch

    scale = 1 / np.sqrt(128)
    ws = gpu.attention_workspace(64, 8)
    for i, (Hq, M, offset) in enumerate([(32, 1, 4000), (32, 1, 10), (64, 5, 700), (64, 8, 1000), (32, 1, 3)]):
        cap = offset + M + 1
        q = gpu.fill_normal_bf16(40 + i, (Hq, M, 128))
        kc = gpu.fill_normal_bf16(50 + i, (8, cap, 128))
        vc = gpu.fill_normal_bf16(60 + i, (8, cap, 128))
        y = gpu.attention(q, kc, vc, offset, scale, workspace=ws)
        ref = orc.sdpa(torch_bf16_bits(q), torch_bf16_bits(kc), torch_bf16_bits(vc), offset + M, offset, M > 1,
                       np.float32(scale))
        assert _close(torch_bf16_bits(y), ref, ulps=2, floor=2e-3) > 0.999, (Hq, M, offset)
    torch.cuda.synchronize()
    assert not ws[:1024].any()  # counters


# (Hq, Hkv, M, offset): decode at several context lengths, new keys straddling
# a 256-key split boundary (253 + 5), 16 new tokens with 4 q heads per kv head
# (64 rows, four row tiles), rep 8 verify
@pytest.mark.parametrize("Hq,Hkv,M,offset", [(32, 8, 1, 0), (32, 8, 1, 4095), (32, 8, 1, 300), (64, 8, 5, 2043),
                                             (32, 8, 5, 253), (32, 8, 16, 100), (16, 8, 3, 511)])
def test_qk_norm_rope_kv_attention_fused(gpu, orc, Hq, Hkv, M, offset):
    """The fused kernel against the two-call sequence (bit-identical out and
    cache rows), twice in a row on one workspace, and against the oracle."""
    import torch

    cap = offset + 2 * M + 3
    kc0 = gpu.fill_normal_bf16(20, (Hkv, cap, 128))
    vc0 = gpu.fill_normal_bf16(21, (Hkv, cap, 128))
    qn = gpu.fill_normal_bf16(22, (128,), sigma=0.3)
    kn = gpu.fill_normal_bf16(23, (128,), sigma=0.3)
    kc_a, vc_a = kc0.clone(), vc0.clone()
    kc_b, vc_b = kc0.clone(), vc0.clone()
    ws = gpu.attention_workspace(Hq, M)
    for step in range(2):
        off = offset + step * M
        q = gpu.fill_normal_bf16(24 + step, (M, Hq * 128), sigma=3.0)
        k = gpu.fill_normal_bf16(26 + step, (M, Hkv * 128), sigma=3.0)
        v = gpu.fill_normal_bf16(28 + step, (M, Hkv * 128))
        qr = gpu.qk_norm_rope_kv(q, k, v, qn, kn, kc_a, vc_a, off)
        y_a = gpu.attention(qr, kc_a, vc_a, off)
        y_b = gpu.qk_norm_rope_kv_attention(q, k, v, qn, kn, kc_b, vc_b, off, workspace=ws)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(torch_bf16_bits(y_b), torch_bf16_bits(y_a))
        np.testing.assert_array_equal(torch_bf16_bits(kc_b), torch_bf16_bits(kc_a))
        np.testing.assert_array_equal(torch_bf16_bits(vc_b), torch_bf16_bits(vc_a))
        ref = orc.sdpa(torch_bf16_bits(qr), torch_bf16_bits(kc_a), torch_bf16_bits(vc_a), off + M, off, M > 1,
                       np.float32(1 / np.sqrt(128)))
        assert _close(torch_bf16_bits(y_b), ref, ulps=2, floor=2e-3) > 0.999
    assert not ws[:1024].any()  # counters back at zero


@pytest.mark.parametrize("M,offset", [(1, 300), (5, 253), (3, 0)])
def test_qk_norm_rope_kv_attention_stale_nan_rows(gpu, M, offset):
    """Cache rows from the new positions on hold NaN (never written memory):
    the fused kernel reads those rows before it writes them, and positions past
    the context are clamped onto them; neither may leak into the output."""
    import torch

    Hq, Hkv = 32, 8
    cap = offset + M + 40
    kc = gpu.fill_normal_bf16(60, (Hkv, cap, 128))
    vc = gpu.fill_normal_bf16(61, (Hkv, cap, 128))
    kc[:, offset:] = float("nan")
    vc[:, offset:] = float("nan")
    kc_a, vc_a = kc.clone(), vc.clone()
    q = gpu.fill_normal_bf16(62, (M, Hq * 128), sigma=3.0)
    k = gpu.fill_normal_bf16(63, (M, Hkv * 128), sigma=3.0)
    v = gpu.fill_normal_bf16(64, (M, Hkv * 128))
    n = gpu.fill_normal_bf16(65, (128,), sigma=0.3)
    y_a = gpu.attention(gpu.qk_norm_rope_kv(q, k, v, n, n, kc_a, vc_a, offset), kc_a, vc_a, offset)
    y_b = gpu.qk_norm_rope_kv_attention(q, k, v, n, n, kc, vc, offset)
    torch.cuda.synchronize()
    assert not torch.isnan(y_b.float()).any()
    np.testing.assert_array_equal(torch_bf16_bits(y_b), torch_bf16_bits(y_a))


def test_qk_norm_rope_kv_attention_limits(gpu):
    import torch

    q = gpu.fill_normal_bf16(30, (17, 32 * 128))
    k = gpu.fill_normal_bf16(31, (17, 8 * 128))
    kc = torch.zeros(8, 64, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    n = gpu.fill_normal_bf16(32, (128,))
    with pytest.raises(gpu.BmxError) as ei:  # 17 new tokens: more than the fused prologue takes
        gpu.qk_norm_rope_kv_attention(q, k, k, n, n, kc, vc, 0)
    assert ei.value.code == gpu.BMX_E_UNSUPPORTED
    with pytest.raises(gpu.BmxError) as ei:
        gpu.qk_norm_rope_kv_attention(q[:4], k[:4], k[:4], n, n, kc, vc, 61)
    assert ei.value.code == gpu.BMX_E_KV_CAPACITY
    torch.cuda.synchronize()
    assert not kc.any() and not vc.any()


@pytest.mark.parametrize("n", [151936, 1001])
def test_argmax(gpu, orc, n):
    """16-byte vector path (rows of a multiple of 8) and the scalar path."""
    x = gpu.fill_normal_bf16(14, (6, n))
    xb = torch_bf16_bits(x).copy()
    xb[1, 7] = xb[1, n - 936] = orc.f32_to_bf16(np.array([30.0], np.float32))[0]
    xb[2, :] = 0x3F80
    xb[3, :] = 0xFF80  # -inf row: index 0
    got = gpu.argmax_rows(to_torch_bf16(xb)).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), orc.argmax_rows(xb))
    assert got[1] == 7 and got[2] == 0 and got[3] == 0


def test_silu_mul_and_add(gpu, orc):
    g = gpu.fill_normal_bf16(15, (3, 9728), sigma=3.0)
    u = gpu.fill_normal_bf16(16, (3, 9728))
    y = torch_bf16_bits(gpu.silu_mul(g, u))
    ref = orc.silu_mul(torch_bf16_bits(g), torch_bf16_bits(u))
    assert np.max(bf16_ulp_diff(y, ref)) <= 1
    s = torch_bf16_bits(gpu.add(g, u))
    np.testing.assert_array_equal(s, orc.f32_to_bf16(bf16_to_f32(torch_bf16_bits(g)) + bf16_to_f32(torch_bf16_bits(u))))


@pytest.mark.parametrize("M,N,K", [(9, 256, 2560), (16, 1024, 2560), (64, 4096, 2560), (128, 2560, 9728),
                                   (300, 1000, 1024), (37, 151936, 2560), (520, 768, 1536), (24, 512, 320),
                                   (130, 300, 576), (1100, 1024, 1536)])
def test_qmm_vs_oracle(gpu, orc, M, N, K):
    import torch

    print(f"qmm M={M} N={N} K={K}", flush=True)
    w, s, b = gpu.init_qlinear(7000 + M, N, K)
    x = gpu.fill_normal_bf16(8000 + M, (M, K))
    y = gpu.quantized_matmul(x, w, s, b)
    torch.cuda.synchronize()
    xb, wq, sb, bb = torch_bf16_bits(x), u32_of(w), torch_bf16_bits(s), torch_bf16_bits(b)
    ref64 = orc.qmatmul_f64(xb, wq, sb, bb)
    yb = torch_bf16_bits(y)
    assert max_rel_err(bf16_to_f32(yb), ref64) < 1e-2
    # the matrix path of the oracle (bf16-dequantized weights, fp32
    # accumulation): within 2 bf16 ulps of it
    assert _close(yb, orc.qmm_dequant(xb, wq, sb, bb), ulps=2, floor=1e-4) == 1.0


@pytest.mark.parametrize("M,N,K", [(64, 1024, 2560), (24, 768, 2048), (16, 2048, 4096), (5, 5120, 8192),
                                   (1, 4096, 2560)])
def test_qmatmul_ws_matches_qmatmul(gpu, M, N, K):
    """bmx_qmatmul_affine_ws with a workspace of exactly
    bmx_qmatmul_workspace_bytes(M, N, K) bytes gives the bits of
    bmx_qmatmul_affine (same kernels, caller-owned partials), and also when
    captured into a graph and replayed."""
    import torch

    print(f"qmatmul_ws M={M} N={N} K={K}", flush=True)
    w, s, b = gpu.init_qlinear(310 + M, N, K)
    x = gpu.fill_normal_bf16(410 + M, (M, K))
    need = gpu.qmatmul_workspace_bytes(M, N, K)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda") if need else None
    ref = gpu.quantized_matmul(x, w, s, b)
    got = gpu.quantized_matmul_ws(x, w, s, b, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(torch_bf16_bits(got), torch_bf16_bits(ref))
    st = torch.cuda.Stream()
    out = torch.empty_like(ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            gpu.quantized_matmul_ws(x, w, s, b, ws, out=out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(torch_bf16_bits(out), torch_bf16_bits(ref))
