"""Pins the oracle's Qwen3 forward / cache / decoding loops:

* against HF transformers' Qwen3ForCausalLM (a third-party implementation
  of the same architecture) running in float32 on the dequantized weights;
* exact invariants of the reference's semantics: forward_multi rows equal
  token-by-token forwards over the cache (causal_mask_offset, RoPE offset,
  slice_update, qwen3.rs:314-563); truncate + replay reproduces logits
  (qwen3.rs:150-161); KV overflow is an error (qwen3.rs:423-428);
  greedy speculative decoding emits exactly the target's greedy tokens
  (speculative.rs:1-24 "exact, no quality loss").
"""
import numpy as np
import pytest
import torch

from _util import bf16_to_f32, max_rel_err

TINY = dict(hidden=256, inter=512, layers=2, n_heads=4, n_kv_heads=2, head_dim=128, vocab=512)


def tiny(orc, seed=1, **kw):
    cfg = orc.make_config(**{**TINY, **kw})
    return orc.Qwen3(cfg, seed, sigma=0.02)


def test_forward_multi_rows_equal_sequential_forwards(orc):
    m = tiny(orc)
    toks = orc.fill_tokens(9, 12, 512)
    c1 = m.new_cache(64)
    multi = m.forward(c1, toks[:7], all_logits=True)
    more = m.forward(c1, toks[7:], all_logits=True)  # offset > 0, M > 1
    c2 = m.new_cache(64)
    seq = np.stack([m.forward(c2, toks[i:i + 1]) for i in range(12)])
    np.testing.assert_array_equal(np.concatenate([multi, more]), seq)
    assert c1.seq_len == c2.seq_len == 12
    np.testing.assert_array_equal(c1.data(), c2.data())


def test_truncate_then_replay_reproduces_logits(orc):
    m = tiny(orc)
    toks = orc.fill_tokens(10, 10, 512)
    c = m.new_cache(32)
    m.forward(c, toks[:6])
    a = m.forward(c, toks[6:], all_logits=True)
    c.truncate(6)
    assert c.seq_len == 6
    c.truncate(8)  # no-op when target >= seq_len
    assert c.seq_len == 6
    b = m.forward(c, toks[6:], all_logits=True)
    np.testing.assert_array_equal(a, b)


def test_kv_capacity_error_leaves_cache(orc):
    m = tiny(orc)
    c = m.new_cache(8)
    m.forward(c, orc.fill_tokens(1, 6, 512))
    snap = c.data().copy()
    with pytest.raises(RuntimeError):
        m.forward(c, orc.fill_tokens(2, 3, 512))
    assert c.seq_len == 6
    np.testing.assert_array_equal(c.data(), snap)


NORM_NAMES = ["input_layernorm", "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm"]


def _random_norms(orc, m, cfg, seed):
    """Fills every norm of the oracle model with its own random weights in
    [0.25, 2] (bf16), so that two norms swapped, or a norm left at 1, change
    the logits."""
    rng = np.random.default_rng(seed)
    for l in list(range(cfg.layers)) + [-1]:
        for which in (range(4) if l >= 0 else (0,)):
            v = m.norm(l, which)
            v[:] = orc.f32_to_bf16(rng.uniform(0.25, 2.0, v.size).astype(np.float32))


def _hf_model(orc, m, cfg, norm_map=None):
    """HF Qwen3ForCausalLM in float32 on the oracle's dequantized weights and
    norm weights.  norm_map(l, which) -> (l', which') wires HF's norm
    (l, which) to the oracle's (l', which') instead (layer -1: final norm),
    for the negative controls."""
    from transformers import Qwen3Config, Qwen3ForCausalLM

    hc = Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                     num_hidden_layers=cfg.layers, num_attention_heads=cfg.n_heads,
                     num_key_value_heads=cfg.n_kv_heads, head_dim=cfg.head_dim, rope_theta=cfg.rope_theta,
                     rms_norm_eps=cfg.eps, tie_word_embeddings=True, max_position_embeddings=4096,
                     attention_bias=False)
    hf = Qwen3ForCausalLM(hc).float().eval()

    def deq(layer, slot):
        w, s, b = m.qlinear(layer, slot)
        return torch.from_numpy(bf16_to_f32(orc.dequantize(w, s, b)))

    def norm(layer, which):
        src = norm_map(layer, which) if norm_map else (layer, which)
        return torch.from_numpy(bf16_to_f32(m.norm(*src)).copy())

    sd = {"model.embed_tokens.weight": deq(-1, 0), "model.norm.weight": norm(-1, 0)}
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.up_proj", "mlp.down_proj"]
    for l in range(cfg.layers):
        for sl, n in enumerate(names):
            sd[f"model.layers.{l}.{n}.weight"] = deq(l, sl)
        for which, n in enumerate(NORM_NAMES):
            sd[f"model.layers.{l}.{n}.weight"] = norm(l, which)
    with torch.no_grad():
        for k, p in hf.named_parameters():
            if k in sd:
                p.copy_(sd[k])
            elif k != "lm_head.weight":
                raise AssertionError(f"unmapped parameter {k}")
        hf.tie_weights()
    return hf


def _hf_errors(orc, m, cfg, toks, norm_map=None):
    hf = _hf_model(orc, m, cfg, norm_map)
    with torch.no_grad():
        ref = hf(torch.from_numpy(toks.astype(np.int64))[None]).logits[0].double().numpy()
    got = bf16_to_f32(m.forward(m.new_cache(32), toks, all_logits=True)).astype(np.float64)
    errs = np.array([max_rel_err(got[t], ref[t]) for t in range(len(toks))])
    return errs, float(np.mean(np.argmax(got, 1) == np.argmax(ref, 1)))


def test_forward_matches_transformers_qwen3(orc):
    """The oracle's forward against HF's, every norm weight random and
    distinct: each position within 3e-2 and >= 80% top-1 agreement."""
    m = tiny(orc, seed=3)
    cfg = m.cfg
    _random_norms(orc, m, cfg, 17)
    toks = orc.fill_tokens(11, 16, cfg.vocab)
    errs, agree = _hf_errors(orc, m, cfg, toks)
    print(f"oracle vs HF Qwen3 (random norms): max rel err {errs.max():.2e}, top-1 {agree:.3f}")
    assert (errs < 3e-2).all(), errs
    assert agree >= 0.8


@pytest.mark.parametrize("swap", ["q_k", "input_post", "final_input0", "layers"])
def test_transformers_pin_detects_swapped_norms(orc, swap):
    """Negative controls of the pin above: the same comparison with two of
    HF's norm weights wired the other way round fails its bar, so a swap in
    the oracle's norm wiring could not pass it either."""
    m = tiny(orc, seed=3)
    cfg = m.cfg
    _random_norms(orc, m, cfg, 17)
    toks = orc.fill_tokens(11, 16, cfg.vocab)
    maps = {
        "q_k": lambda l, w: (l, {2: 3, 3: 2}.get(w, w)) if l >= 0 else (l, w),
        "input_post": lambda l, w: (l, {0: 1, 1: 0}.get(w, w)) if l >= 0 else (l, w),
        "final_input0": lambda l, w: (0, 0) if l < 0 else ((-1, 0) if (l, w) == (0, 0) else (l, w)),
        "layers": lambda l, w: ((1 - l), w) if l >= 0 else (l, w),
    }
    errs, _ = _hf_errors(orc, m, cfg, toks, maps[swap])
    print(f"swapped norms ({swap}): max rel err {errs.max():.2e}")
    assert errs.max() > 3e-2, errs


def test_greedy_generate_follows_forward(orc):
    m = tiny(orc, seed=4)
    prompt = orc.fill_tokens(12, 8, 512)
    c = m.new_cache(64)
    out = orc.generate_greedy(m, c, prompt, 10, eos=())
    assert len(out) == 10
    # replay: each emitted token is the argmax of the forward that preceded it
    c2 = m.new_cache(64)
    logits = m.forward(c2, prompt)
    for t in out:
        assert int(np.argmax(bf16_to_f32(logits))) == t
        logits = m.forward(c2, [t])


def test_speculative_emits_the_greedy_tokens(orc):
    target = tiny(orc, seed=5)
    draft = tiny(orc, seed=6, layers=1)
    prompt = orc.fill_tokens(13, 8, 512)
    greedy = orc.generate_greedy(target, target.new_cache(128), prompt, 24, eos=())
    spec, stats = orc.speculative_generate(target, target.new_cache(128), draft, draft.new_cache(128), prompt, 24,
                                           spec_k=5, eos=())
    np.testing.assert_array_equal(spec, greedy)
    assert stats[0] > 0 and stats[1] >= stats[2]
    # a draft identical to the target is always accepted
    twin = tiny(orc, seed=5)
    spec2, stats2 = orc.speculative_generate(target, target.new_cache(128), twin, twin.new_cache(128), prompt, 24,
                                             spec_k=5, eos=())
    np.testing.assert_array_equal(spec2, greedy)
    assert stats2[1] == stats2[2] and stats2[1] > 0
