"""GPU parity of gather_qmm (routed MoE expert qmm) against the CPU oracle:
within 2 bf16 ulps of the oracle's fp32-accumulated result per route, for
the Qwen3-30B-A3B-shaped decode projections (128 experts of gate|up
(1536, 2048) with x shared over the 8 routes of a token, down (2048, 768)
with one x block per route), ragged shapes, several rows of x per route,
repeated and out-of-range expert ids."""
import numpy as np
import pytest

from _util import bf16_to_f32, to_torch_bf16, torch_bf16_bits, u32_of

pytestmark = pytest.mark.gpu


def _experts(gpu, orc, seed, E, N, K):
    import torch

    dev = [gpu.init_qlinear(seed + e, N, K) for e in range(E)]
    w, s, b = (torch.stack([t[i] for t in dev]).contiguous() for i in range(3))
    return (w, s, b), (u32_of(w), torch_bf16_bits(s), torch_bf16_bits(b))


def _close(y_bits, ref_bits):
    y = bf16_to_f32(y_bits).astype(np.float64)
    r = bf16_to_f32(ref_bits).astype(np.float64)
    ok = np.abs(y - r) <= np.maximum(2 * np.abs(r) * 2.0 ** -7, 1e-4 * np.max(np.abs(r)))
    return ok.mean()


# (E, N, K, M, R, x_bcast)
CASES = [(128, 1536, 2048, 1, 8, 8), (128, 2048, 768, 1, 8, 1), (5, 100, 320, 3, 7, 1), (8, 256, 4096, 8, 4, 2),
         (3, 64, 64, 2, 6, 3)]


@pytest.mark.parametrize("E,N,K,M,R,x_bcast", CASES)
def test_gather_qmm(gpu, orc, E, N, K, M, R, x_bcast):
    import torch

    print(f"gather_qmm E={E} N={N} K={K} M={M} R={R} x_bcast={x_bcast}", flush=True)
    (w, s, b), (wq, sq, bq) = _experts(gpu, orc, 1000 + K, E, N, K)
    rng = np.random.default_rng(R * 31 + E)
    rhs = rng.integers(0, E, R).astype(np.uint32)
    rhs[-1] = rhs[0]  # a repeated expert
    x = gpu.fill_normal_bf16(2000 + M, (R // x_bcast, M, K))
    rhs_d = torch.from_numpy(rhs.view(np.int32)).cuda()
    y = gpu.gather_qmm(x, w, s, b, rhs_d, x_bcast)
    torch.cuda.synchronize()
    ref = orc.gather_qmm(torch_bf16_bits(x), wq, sq, bq, rhs, x_bcast)
    assert _close(torch_bf16_bits(y), ref) > 0.999
    # out-of-range ids: clamped to the last expert
    rhs2 = rhs.copy()
    rhs2[0] = E + 5
    y2 = gpu.gather_qmm(x, w, s, b, torch.from_numpy(rhs2.view(np.int32)).cuda(), x_bcast)
    rhs2[0] = E - 1
    y3 = gpu.gather_qmm(x, w, s, b, torch.from_numpy(rhs2.view(np.int32)).cuda(), x_bcast)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(torch_bf16_bits(y2), torch_bf16_bits(y3))


def test_gather_qmm_matches_qmatmul_per_route(gpu, orc):
    """A single route with x_bcast 1 is the plain quantized_matmul of its expert."""
    import torch

    E, N, K = 4, 384, 1024
    (w, s, b), _ = _experts(gpu, orc, 3000, E, N, K)
    x = gpu.fill_normal_bf16(3100, (1, 1, K))
    for e in range(E):
        y = gpu.gather_qmm(x, w, s, b, torch.tensor([e], dtype=torch.int32, device="cuda"))
        z = gpu.quantized_matmul(x[0], w[e], s[e], b[e])
        torch.cuda.synchronize()
        assert _close(torch_bf16_bits(y[0]), torch_bf16_bits(z)) == 1.0


def test_gather_qmm_errors(gpu):
    import torch

    w = torch.zeros(2, 16, 8, dtype=torch.int32, device="cuda")
    s = torch.zeros(2, 16, 1, dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(1, 9, 64, dtype=torch.bfloat16, device="cuda")
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(gpu.BmxError) as ei:  # 9 rows of x per route
        gpu.gather_qmm(x, w, s, s, idx)
    assert ei.value.code == gpu.BMX_E_UNSUPPORTED


def test_gather_qmm_indexed_lhs_and_rhs(gpu, orc):
    """mlx_gather_qmm with both index arrays: route r multiplies x block
    lhs[r] (repeated, permuted and one out-of-range id, clamped to the last
    block) by expert rhs[r]; checked against the oracle run on the x blocks
    gathered on the host."""
    import torch

    E, N, K, M, B, R = 6, 320, 1536, 2, 5, 9
    print(f"gather_qmm_indexed E={E} N={N} K={K} M={M} x blocks={B} R={R}", flush=True)
    (w, s, b), (wq, sq, bq) = _experts(gpu, orc, 4000, E, N, K)
    rng = np.random.default_rng(17)
    lhs = rng.integers(0, B, R).astype(np.uint32)
    lhs[2] = B + 3  # clamped to B - 1
    rhs = rng.integers(0, E, R).astype(np.uint32)
    x = gpu.fill_normal_bf16(4100, (B, M, K))
    dev = lambda a: torch.from_numpy(a.view(np.int32)).cuda()  # noqa: E731
    y = gpu.gather_qmm_indexed(x, w, s, b, dev(lhs), dev(rhs), sorted_indices=True)
    torch.cuda.synchronize()
    xg = torch_bf16_bits(x)[np.minimum(lhs, B - 1)]
    ref = orc.gather_qmm(xg, wq, sq, bq, rhs, 1)
    assert _close(torch_bf16_bits(y), ref) > 0.999
    # without lhs_indices the x blocks broadcast over the routes: the same
    # bits as bmx_gather_qmm with x_bcast = R / B
    x3 = gpu.fill_normal_bf16(4200, (3, M, K))
    rhs6 = dev(rng.integers(0, E, 6).astype(np.uint32))
    a = gpu.gather_qmm_indexed(x3, w, s, b, None, rhs6)
    c = gpu.gather_qmm(x3, w, s, b, rhs6, x_bcast=2)
    # without rhs_indices route r uses expert r (R = E)
    x6 = gpu.fill_normal_bf16(4300, (E, M, K))
    d = gpu.gather_qmm_indexed(x6, w, s, b, None, None)
    e = gpu.gather_qmm(x6, w, s, b, dev(np.arange(E, dtype=np.uint32)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(torch_bf16_bits(a), torch_bf16_bits(c))
    np.testing.assert_array_equal(torch_bf16_bits(d), torch_bf16_bits(e))


def test_gather_qmm_indexed_errors(gpu):
    import torch

    w = torch.zeros(2, 16, 8, dtype=torch.int32, device="cuda")
    s = torch.zeros(2, 16, 1, dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(3, 1, 64, dtype=torch.bfloat16, device="cuda")
    idx = torch.zeros(4, dtype=torch.int32, device="cuda")
    cases = [(dict(lhs_indices=idx, rhs_indices=idx, transpose=False), gpu.BMX_E_UNSUPPORTED),
             (dict(lhs_indices=None, rhs_indices=idx), gpu.BMX_E_SHAPE),  # 4 routes over 3 x blocks
             (dict(lhs_indices=idx, rhs_indices=None), gpu.BMX_E_SHAPE)]  # 4 routes, 2 experts
    for kw, code in cases:
        with pytest.raises(gpu.BmxError) as ei:
            gpu.gather_qmm_indexed(x, w, s, s, **kw)
        assert ei.value.code == code, kw
