"""MLX checkpoints through the loader on the GPU: a checkpoint exported from
the random-init GPU model loads bit-identical (same logits bits), and a
checkpoint of the oracle's weights with non-trivial norm weights (stored as
F32, two shards, `quantization_config` only, untied head) reproduces the
oracle's forward within the end-to-end bar (2e-2 relative, greedy top-1)."""
import numpy as np
import pytest

from _ckpt import model_tensors, write_model
from _util import bf16_to_f32, l2_rel_err, torch_bf16_bits

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=512, inter=1536, layers=3, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)


def test_load_export_of_random_model_bit_identical(gpu, orc, tmp_path):
    import torch

    gm = gpu.Qwen3(gpu.qwen3_config(**SMALL), 11, 0.02, max_tokens=32)
    ones = lambda layer, which: np.full(128 if (layer >= 0 and which >= 2) else SMALL["hidden"], 0x3F80, np.uint16)
    t = model_tensors({**SMALL, "tied": 1}, gm.qlinear_numpy, ones)
    write_model(str(tmp_path / "ck"), {**SMALL, "tied": 1}, t, shards=2)
    lm = gpu.Qwen3.load(str(tmp_path / "ck"), max_tokens=32)
    assert (lm.cfg.hidden, lm.cfg.layers, lm.cfg.vocab, lm.cfg.tied) == (512, 3, 4096, 1)
    for layer, slot in [(-1, 0)] + [(l, s) for l in range(SMALL["layers"]) for s in range(7)]:
        for name, x, y in zip("wsb", gm.qlinear_numpy(layer, slot), lm.qlinear_numpy(layer, slot)):
            np.testing.assert_array_equal(x, y, err_msg=f"layer {layer} slot {slot} {name}")
    toks = orc.fill_tokens(5, 9, SMALL["vocab"])
    ga, la = gm.new_cache(64), lm.new_cache(64)
    a = gm.forward(ga, toks, all_logits=True)
    b = lm.forward(la, toks, all_logits=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(torch_bf16_bits(a), torch_bf16_bits(b))
    assert gm.decode_step(ga, 17) == lm.decode_step(la, 17)


def test_load_oracle_weights_with_norms(gpu, orc, tmp_path):
    import torch

    shape = {**SMALL, "tied": 0}
    om = orc.Qwen3(orc.make_config(**shape), 21, 0.02)
    rng = np.random.default_rng(3)
    for layer in list(range(shape["layers"])) + [-1]:
        for which in (range(4) if layer >= 0 else [0]):
            v = om.norm(layer, which)
            v[:] = orc.f32_to_bf16(rng.normal(1.0, 0.25, v.size).astype(np.float32))
    t = model_tensors(shape, om.qlinear, om.norm, norm_dtype="F32")
    write_model(str(tmp_path / "ck"), shape, t, shards=2, quant_key="quantization_config")
    gm = gpu.Qwen3.load(str(tmp_path / "ck"), max_tokens=32)
    assert gm.cfg.tied == 0
    toks = orc.fill_tokens(6, 20, shape["vocab"])
    gc, oc = gm.new_cache(64), om.new_cache(64)
    g = gm.forward(gc, toks, all_logits=True)
    o = om.forward(oc, toks, all_logits=True)
    torch.cuda.synchronize()
    gf = bf16_to_f32(torch_bf16_bits(g)).astype(np.float64)
    of = bf16_to_f32(o).astype(np.float64)
    errs = [l2_rel_err(a, b) for a, b in zip(gf, of)]
    agree = np.mean(np.argmax(gf, 1) == np.argmax(of, 1))
    print(f"loaded vs oracle: max rel err {max(errs):.2e}, top-1 agreement {agree:.3f}", flush=True)
    assert max(errs) < 2e-2 and agree >= 0.9
    # the norms matter: the same weights with unit norms give other logits
    gr = gpu.Qwen3(gpu.qwen3_config(**shape), 21, 0.02, max_tokens=32)
    r = gr.forward(gr.new_cache(64), toks, all_logits=True)
    torch.cuda.synchronize()
    assert l2_rel_err(bf16_to_f32(torch_bf16_bits(r)).astype(np.float64), of) > 5e-2
