"""GPU parity of the quantized-matmul path against the CPU oracle.

* seeded init and dequantization: bit-exact (integer / byte work);
* qmv (M <= 8): within max relative error 1e-2 of the float64 product
  (bf16 out, fp32 accumulate) and within 2 bf16 ulps of the oracle's own
  fp32-accumulated result.
"""
import numpy as np
import pytest

from _util import bf16_to_f32, max_rel_err, to_torch_bf16, torch_bf16_bits, u32_of

pytestmark = pytest.mark.gpu

QWEN3_4B_QMV = [(4096, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (2560, 9728), (151936, 2560)]


def _close_to_oracle(y_bits, ref_bits):
    y = bf16_to_f32(y_bits).astype(np.float64)
    r = bf16_to_f32(ref_bits).astype(np.float64)
    ulp = np.abs(r) * 2.0 ** -7
    ok = np.abs(y - r) <= np.maximum(2 * ulp, 1e-4 * np.max(np.abs(r)))
    return ok.mean(), np.max(np.abs(y - r))


def test_init_qlinear_bit_exact(gpu, orc):
    for seed, (N, K) in [(1, (37, 64)), (2, (256, 2560)), (3, (1024, 9728))]:
        print(f"init N={N} K={K}", flush=True)
        w, s, b = gpu.init_qlinear(seed, N, K)
        wq, sq, bq = orc.init_qlinear(seed, N, K)
        np.testing.assert_array_equal(u32_of(w), wq)
        np.testing.assert_array_equal(torch_bf16_bits(s), sq)
        np.testing.assert_array_equal(torch_bf16_bits(b), bq)


def test_fill_normal_bit_exact(gpu, orc):
    x = gpu.fill_normal_bf16(42, (3, 1000), sigma=1.0)
    np.testing.assert_array_equal(torch_bf16_bits(x).ravel(), orc.fill_normal_bf16(42, 3000, sigma=1.0))


def test_dequantize_and_gather_bit_exact(gpu, orc):
    import torch

    w, s, b = gpu.init_qlinear(5, 300, 1024)
    wq, sq, bq = orc.init_qlinear(5, 300, 1024)
    np.testing.assert_array_equal(torch_bf16_bits(gpu.dequantize(w, s, b)), orc.dequantize(wq, sq, bq))
    ids = np.array([0, 299, 17, 17, 150], np.int32)
    got = gpu.dequant_gather(torch.from_numpy(ids).cuda(), w, s, b)
    np.testing.assert_array_equal(torch_bf16_bits(got), orc.dequant_gather(ids.astype(np.uint32), wq, sq, bq))
    # an out-of-range id yields a zero row (documented in include/bmx.h)
    bad = gpu.dequant_gather(torch.tensor([300, -1], dtype=torch.int32, device="cuda"), w, s, b)
    assert torch.count_nonzero(bad.float()).item() == 0


def _check_qmv(gpu, orc, M, N, K, seed):
    import torch

    print(f"qmv M={M} N={N} K={K}", flush=True)
    w, s, b = gpu.init_qlinear(seed, N, K)
    x = gpu.fill_normal_bf16(seed + 1, (M, K), sigma=1.0)
    y = gpu.quantized_matmul(x, w, s, b)
    torch.cuda.synchronize()
    wq, sq, bq = u32_of(w), torch_bf16_bits(s), torch_bf16_bits(b)
    xb = torch_bf16_bits(x)
    ref = orc.qmatmul(xb, wq, sq, bq)
    ref64 = orc.qmatmul_f64(xb, wq, sq, bq)
    yb = torch_bf16_bits(y)
    assert max_rel_err(bf16_to_f32(yb), ref64) < 1e-2
    frac, worst = _close_to_oracle(yb, ref)
    assert frac == 1.0, (frac, worst)


@pytest.mark.parametrize("N,K", QWEN3_4B_QMV)
def test_qmv_qwen3_4b_shapes(gpu, orc, N, K):
    _check_qmv(gpu, orc, 1, N, K, seed=1000 + N + K)


@pytest.mark.parametrize("M", [2, 3, 4, 5, 6, 7, 8])
def test_qmv_multi_row(gpu, orc, M):
    _check_qmv(gpu, orc, M, 1024, 2560, seed=3000 + M)


@pytest.mark.parametrize("N,K", [(1, 64), (37, 64), (100, 192), (513, 3072), (2048, 1024), (1024, 25600)])
def test_qmv_edge_shapes(gpu, orc, N, K):
    _check_qmv(gpu, orc, 1, N, K, seed=5000 + N)
    _check_qmv(gpu, orc, 5, N, K, seed=6000 + N)


@pytest.mark.parametrize("M,N,K", [(5, 5120, 8192), (8, 4096, 12288), (2, 1320, 25600), (3, 4104, 8192)])
def test_qmv_split_k(gpu, orc, M, N, K):
    """Shapes whose matrix-core GEMV splits K over workgroups (fp32 partials
    reduced by a second launch), including a row count that leaves a partial
    16-row tile."""
    _check_qmv(gpu, orc, M, N, K, seed=7000 + M + N)


def test_qmv_integer_exact(gpu, orc):
    """s = b = 1 and x in {-1,0,1}: every output is an exact small integer."""
    import torch

    rng = np.random.default_rng(7)
    N, K, M = 96, 2560, 3
    q = rng.integers(0, 16, (N, K)).astype(np.uint32)
    wq = np.bitwise_or.reduce(q.reshape(N, K // 8, 8) << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)
    xi = rng.integers(-1, 2, (M, K))
    xs = orc.f32_to_bf16(xi.astype(np.float32))
    one = np.full((N, K // 64), 0x3F80, np.uint16)
    y = gpu.quantized_matmul(to_torch_bf16(xs), torch.from_numpy(wq.view(np.int32)).cuda(), to_torch_bf16(one),
                             to_torch_bf16(one))
    ref = xi @ (q.astype(np.int64) + 1).T
    got = bf16_to_f32(torch_bf16_bits(y))
    small = np.abs(ref) <= 256
    np.testing.assert_array_equal(got[small], ref[small].astype(np.float32))


def test_qmv_linearity_full_lm_head(gpu, orc):
    """Size-independent properties at the full lm_head shape (151936 x 2560):
    y(2x) == 2 y(x) bit for bit (power-of-two scaling is exact through the
    fp32 accumulation), and y(x1 + x2) = y(x1) + y(x2) for disjoint supports."""
    import torch

    N, K = 151936, 2560
    w, s, b = gpu.init_qlinear(11, N, K)
    x = gpu.fill_normal_bf16(12, (1, K))
    y1 = gpu.quantized_matmul(x, w, s, b)
    y2 = gpu.quantized_matmul((x.float() * 2).to(torch.bfloat16), w, s, b)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(torch_bf16_bits((y1.float() * 2).to(torch.bfloat16)), torch_bf16_bits(y2))
    even = torch.zeros_like(x)
    odd = torch.zeros_like(x)
    even[:, 0::2] = x[:, 0::2]
    odd[:, 1::2] = x[:, 1::2]
    ye = gpu.quantized_matmul(even, w, s, b).float()
    yo = gpu.quantized_matmul(odd, w, s, b).float()
    torch.cuda.synchronize()
    assert max_rel_err((ye + yo).cpu().numpy(), y1.float().cpu().numpy()) < 1e-2


@pytest.mark.parametrize("N,K", [(4096, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (2560, 9728),
                                 (151936, 2560), (10240, 5120), (5120, 8192), (5120, 25600), (576, 320)])
def test_gemv_rows_independent_of_row_count(gpu, N, K):
    """Each row of an M-row GEMV (M = 2..8) has the bits of the same row
    computed alone: the single-phase, persistent and phased kernels share one
    per-row arithmetic, and the lanes per weight row depend on N and K only
    (this is what makes greedy speculative decoding exact)."""
    import torch

    print(f"row invariance N={N} K={K}", flush=True)
    w, s, b = gpu.init_qlinear(4000 + N % 97, N, K)
    x = gpu.fill_normal_bf16(4100 + K % 89, (8, K))
    singles = [torch_bf16_bits(gpu.quantized_matmul(x[i:i + 1], w, s, b)) for i in range(8)]
    for M in range(2, 9):
        y = torch_bf16_bits(gpu.quantized_matmul(x[:M].contiguous(), w, s, b))
        for i in range(M):
            np.testing.assert_array_equal(y[i], singles[i][0], err_msg=f"M={M} row {i}")
