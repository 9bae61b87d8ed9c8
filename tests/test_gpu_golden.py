"""The HIP path against the committed golden fixtures (tests/golden/,
closed forms in float64): dyadic quantized matmuls bit-exact through both
the GEMV (M <= 8) and the MFMA GEMM (M = 12), dequantized weights and the
nibble order bit-exact, random small matmuls within 1e-2 of float64, RoPE
within 2 bf16 ulps, the KV slice write bit-exact."""
import os

import numpy as np
import pytest

from _util import bf16_to_f32, bf16_ulp_diff, max_rel_err, to_torch_bf16, to_torch_u32, torch_bf16_bits

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name))


@pytest.mark.parametrize("i", range(5))
def test_gpu_dyadic_qmatmul_and_dequant_exact(gpu, i):
    d = load("dyadic_qmm.npz")
    x, w, s, b = (to_torch_bf16(d[f"x_{i}"]), to_torch_u32(d[f"w_{i}"]), to_torch_bf16(d[f"s_{i}"]),
                  to_torch_bf16(d[f"b_{i}"]))
    print(f"dyadic case {i}: M={x.shape[0]} N={w.shape[0]} K={x.shape[1]}", flush=True)
    np.testing.assert_array_equal(torch_bf16_bits(gpu.dequantize(w, s, b)), d[f"deq_{i}"])
    np.testing.assert_array_equal(torch_bf16_bits(gpu.quantized_matmul(x, w, s, b)), d[f"y_{i}"])


def test_gpu_pack_table(gpu):
    d = load("pack_table.npz")
    words = to_torch_u32(d["words"].reshape(32, 8))
    one = to_torch_bf16(np.full((32, 1), 0x3F80, np.uint16))
    zero = to_torch_bf16(np.zeros((32, 1), np.uint16))
    deq = bf16_to_f32(torch_bf16_bits(gpu.dequantize(words, one, zero)))
    np.testing.assert_array_equal(deq.reshape(256, 8), d["nibbles"].astype(np.float32))


@pytest.mark.parametrize("i", range(3))
def test_gpu_tiny_qmatmul_vs_float64(gpu, i):
    d = load("tiny_qmm_f64.npz")
    y = gpu.quantized_matmul(to_torch_bf16(d[f"x_{i}"]), to_torch_u32(d[f"w_{i}"]), to_torch_bf16(d[f"s_{i}"]),
                             to_torch_bf16(d[f"b_{i}"]))
    assert max_rel_err(bf16_to_f32(torch_bf16_bits(y)), d[f"y64_{i}"]) < 1e-2


@pytest.mark.parametrize("offset", [0, 1, 4095])
def test_gpu_rope_fixture(gpu, offset):
    d = load("rope.npz")
    y = gpu.rope(to_torch_bf16(d["x"]), 1e6, offset)
    assert np.max(bf16_ulp_diff(torch_bf16_bits(y), d[f"y_{offset}"])) <= 2


def test_gpu_kv_write_fixture(gpu):
    import torch

    d = load("kv_write.npz")
    src = to_torch_bf16(d["src"])
    gpu.slice_update(src, to_torch_bf16(d["update"]), d["start"].tolist(), d["stop"].tolist(), d["strides"].tolist())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(torch_bf16_bits(src), d["after"])
