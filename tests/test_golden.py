"""The oracle against the committed golden fixtures of tests/golden/, which
tests/golden/make_golden.py computes from closed forms in float64 (numpy
only): exact dyadic quantized matmuls and dequantized weights, the nibble
order of packed words, random small matmuls in float64, RoPE at offsets
0 / 1 / 4095 and a KV-cache slice write at offset cap - M."""
import os

import numpy as np
import pytest

from _util import bf16_to_f32, bf16_ulp_diff, max_rel_err

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name))


@pytest.mark.parametrize("i", range(5))
def test_oracle_dyadic_qmatmul_and_dequant_exact(orc, i):
    d = load("dyadic_qmm.npz")
    x, w, s, b = d[f"x_{i}"], d[f"w_{i}"], d[f"s_{i}"], d[f"b_{i}"]
    np.testing.assert_array_equal(orc.dequantize(w, s, b), d[f"deq_{i}"])
    np.testing.assert_array_equal(orc.qmatmul(x, w, s, b), d[f"y_{i}"])
    np.testing.assert_array_equal(orc.qmatmul_f64(x, w, s, b), d[f"y64_{i}"])


def test_oracle_pack_table(orc):
    d = load("pack_table.npz")
    words = d["words"].reshape(32, 8)  # 32 rows of K = 64
    one = np.full((32, 1), 0x3F80, np.uint16)
    zero = np.zeros((32, 1), np.uint16)
    deq = bf16_to_f32(orc.dequantize(words, one, zero))
    np.testing.assert_array_equal(deq.reshape(256, 8), d["nibbles"].astype(np.float32))


@pytest.mark.parametrize("i", range(3))
def test_oracle_tiny_qmatmul_vs_float64(orc, i):
    d = load("tiny_qmm_f64.npz")
    args = (d[f"x_{i}"], d[f"w_{i}"], d[f"s_{i}"], d[f"b_{i}"])
    assert max_rel_err(bf16_to_f32(orc.qmatmul(*args)), d[f"y64_{i}"]) < 1e-2
    np.testing.assert_allclose(orc.qmatmul_f64(*args), d[f"y64_{i}"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("offset", [0, 1, 4095])
def test_oracle_rope_fixture(orc, offset):
    d = load("rope.npz")
    y = orc.rope(d["x"], 1e6, offset)
    # fp32 rotation with a float frequency table vs float64: at most 1 bf16 ulp
    assert np.max(bf16_ulp_diff(y, d[f"y_{offset}"])) <= 1


def test_oracle_kv_write_fixture(orc):
    d = load("kv_write.npz")
    src = d["src"].copy()
    assert orc.slice_update(src, d["update"], d["start"], d["stop"], d["strides"]) == 0
    np.testing.assert_array_equal(src, d["after"])
