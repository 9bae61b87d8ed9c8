"""Greedy speculative decoding is exact on the GPU.

The reference's algorithm is "greedy variant -- exact, no quality loss"
(crates/base-mlx-core/src/speculative.rs:3-6).  It holds here bit for bit
because a verify forward of M tokens computes every row with the same
operations as a single-token decode of that position: the GEMVs share one
per-row arithmetic whatever M (tests/test_gpu_qmv.py), and decode attention
reduces every query row the same way whatever the tile of rows.  So:
  * the rows of an M-token forward equal M single-token decode steps, logits
    and KV cache rows, bit for bit;
  * speculative output equals greedy output token for token (any draft);
  * against the oracle, the GPU's tokens are the oracle's argmax at every
    step except at near-ties, and it takes no more of those the other way
    than the oracle does against itself with its summation order reversed.
"""
import numpy as np
import pytest

from _parity import BF16_STEPS, FLOOR_FACTOR
from _util import bf16_to_f32, torch_bf16_bits

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=512, inter=1536, layers=3, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)
QWEN3_0_6B = dict(hidden=1024, inter=3072, layers=28, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936)
QWEN3_4B = dict(hidden=2560, inter=9728, layers=36, n_heads=32, n_kv_heads=8, head_dim=128, vocab=151936)
QWEN3_32B = dict(hidden=5120, inter=25600, layers=64, n_heads=64, n_kv_heads=8, head_dim=128, vocab=151936, tied=0)


def _gpu(gpu, shape, seed, max_tokens=64, **kw):
    return gpu.Qwen3(gpu.qwen3_config(**{**shape, **kw}), seed, 0.02, max_tokens=max_tokens)


def _verify_rows_equal_decode_steps(gpu, model, prefill, toks, cap, fill=0):
    """Logits and KV rows of one forward over `toks` == those of len(toks)
    single-token graph decode steps, after the same prefill (or the same
    synthetic fill of `fill` positions)."""
    a, b = model.new_cache(cap), model.new_cache(cap)
    for c in (a, b):
        if fill:
            c.fill_synthetic(77, fill)
        else:
            model.forward(c, prefill)
    p0 = a.seq_len
    steps = [torch_bf16_bits(model.decode_step(a, int(t), want_logits=True)[1]) for t in toks]
    rows = torch_bf16_bits(model.forward(b, toks, all_logits=True))
    for i in range(len(toks)):
        np.testing.assert_array_equal(rows[i], steps[i], err_msg=f"row {i}")
    n = model.cfg.layers
    for layer in sorted({0, n // 2, n - 1}):
        for kv in (0, 1):
            np.testing.assert_array_equal(a.layer_numpy(layer, kv)[:, p0:p0 + len(toks)],
                                          b.layer_numpy(layer, kv)[:, p0:p0 + len(toks)])


@pytest.mark.parametrize("M", [2, 3, 5, 8])
def test_small_verify_rows_equal_decode_steps(gpu, orc, M):
    m = _gpu(gpu, SMALL, 21)
    prompt = orc.fill_tokens(31, 17, SMALL["vocab"])
    _verify_rows_equal_decode_steps(gpu, m, prompt, orc.fill_tokens(32 + M, M, SMALL["vocab"]), 64)


def test_4b_verify_rows_equal_decode_steps(gpu, orc):
    """The Qwen3-4B shape (36 layers): a 5-token verify forward at context
    300 equals five decode steps."""
    m = _gpu(gpu, QWEN3_4B, 42, max_tokens=16)
    _verify_rows_equal_decode_steps(gpu, m, None, orc.fill_tokens(40, 5, QWEN3_4B["vocab"]), 512, fill=300)


def test_32b_shape_verify_rows_equal_decode_steps(gpu, orc):
    """The Qwen3-32B shape (2 of its layers, untied head; K = 25600 down
    projection on the phased GEMV): verify at context 2048 == decode."""
    m = _gpu(gpu, QWEN3_32B, 13, max_tokens=16, layers=2)
    _verify_rows_equal_decode_steps(gpu, m, None, orc.fill_tokens(41, 5, QWEN3_32B["vocab"]), 2304, fill=2048)


def test_small_verify_rows_equal_decode_steps_at_long_context(gpu, orc):
    """An 8-token verify at context 40000 (157 key splits of 256) equals
    eight decode steps: the model's attention workspace holds 256 splits for
    every fused width, so verify rows take the split-key path wherever a
    decode step does."""
    m = _gpu(gpu, SMALL, 23, max_tokens=16)
    _verify_rows_equal_decode_steps(gpu, m, None, orc.fill_tokens(43, 8, SMALL["vocab"]), 40960, fill=40000)


def _spec_equals_greedy(gpu, target, draft, prompt, n, spec_k=5):
    greedy = target.generate_greedy(target.new_cache(len(prompt) + n + 16), prompt, n, eos=())
    spec, stats = gpu.speculative_generate(target, target.new_cache(len(prompt) + n + 16), draft,
                                           draft.new_cache(len(prompt) + n + 16), prompt, n, spec_k=spec_k, eos=())
    print(f"speculative: {len(spec)} tokens, iterations {stats[0]}, drafted {stats[1]}, accepted {stats[2]}",
          flush=True)
    np.testing.assert_array_equal(spec, greedy)
    return greedy, stats


def test_small_speculative_equals_greedy_token_for_token(gpu, orc):
    """3-layer target, 128 tokens, with three drafts: an unrelated 1-layer
    model (nothing accepted), the target's own first layer (a truncated copy:
    some accepted) and an identical twin (all accepted)."""
    target = _gpu(gpu, SMALL, 7)
    prompt = orc.fill_tokens(14, 10, SMALL["vocab"])
    for draft, spec_k in ((_gpu(gpu, SMALL, 8, layers=1), 5), (_gpu(gpu, SMALL, 7, layers=1), 5),
                          (_gpu(gpu, SMALL, 7), 5), (_gpu(gpu, SMALL, 7, layers=2), 3)):
        _, stats = _spec_equals_greedy(gpu, target, draft, prompt, 128, spec_k)
    assert stats[2] > 0


def test_speculative_continues_a_filled_cache(gpu, orc):
    """Caches that already hold context: the rewinds are relative to where
    each cache starts (the oracle does the same), and the result equals
    greedy decoding from that context."""
    target, draft = _gpu(gpu, SMALL, 7), _gpu(gpu, SMALL, 7, layers=1)
    ctx = orc.fill_tokens(50, 20, SMALL["vocab"])
    prompt = orc.fill_tokens(51, 6, SMALL["vocab"])
    tc, dc, gc = target.new_cache(256), draft.new_cache(256), target.new_cache(256)
    target.forward(tc, ctx)
    draft.forward(dc, ctx)
    target.forward(gc, ctx)
    spec, _ = gpu.speculative_generate(target, tc, draft, dc, prompt, 48, spec_k=5, eos=())
    greedy = target.generate_greedy(gc, prompt, 48, eos=())
    np.testing.assert_array_equal(spec, greedy)
    om, odm = orc.Qwen3(orc.make_config(**SMALL), 7, 0.02), orc.Qwen3(orc.make_config(**{**SMALL, "layers": 1}), 7, 0.02)
    otc, odc = om.new_cache(256), odm.new_cache(256)
    om.forward(otc, ctx)
    odm.forward(odc, ctx)
    ospec, _ = orc.speculative_generate(om, otc, odm, odc, prompt, 48, spec_k=5, eos=())
    ogc = om.new_cache(256)
    om.forward(ogc, ctx)
    np.testing.assert_array_equal(ospec, orc.generate_greedy(om, ogc, prompt, 48, eos=()))


def _agree_with_oracle_greedy(orc, om, tokens, prompt, cap, fill=0, fill_seed=0):
    """Teacher-forces the oracle on the GPU's greedy `tokens` (after `prompt`,
    from a cache with `fill` synthetic positions), and beside it the oracle
    with every fp32 reduction reversed.  Per position, a GPU flip is a token
    other than the oracle's argmax; a floor flip is the reversed oracle's
    argmax differing from the oracle's (what summation order alone does on
    the same token stream).  Every GPU flip must be a near-tie: the oracle's
    gap between its argmax and the GPU's token at most BF16_STEPS bf16 steps
    of the top logit, or 4 standard deviations of a difference of two logits
    at the GPU's allowed spread (FLOOR_FACTOR x the position's rms
    reordering spread, times sqrt 2 for the difference).  The rms over the
    vocabulary estimates the spread at the two tokens in question: the GPU's
    deviation at a token is independent of the reversed oracle's deviation
    there, so the latter's value at those two tokens would be a single draw,
    not a bound.  Returns (GPU flips, floor flips, positions)."""
    oc, rc = om.new_cache(cap), om.new_cache(cap)
    if fill:
        oc.fill_synthetic(fill_seed, fill)
        rc.fill_synthetic(fill_seed, fill)
    logits = om.forward(oc, prompt)
    with orc.reversed_accumulation():
        rlogits = om.forward(rc, prompt)
    flips = floor_flips = 0
    for i, t in enumerate(tokens):
        o = bf16_to_f32(logits).astype(np.float64)
        r = bf16_to_f32(rlogits).astype(np.float64)
        a = int(np.argmax(o))
        floor_flips += int(np.argmax(r)) != a
        if a != int(t):
            gap = o[a] - o[int(t)]
            ulp = 2.0 ** (np.floor(np.log2(abs(o[a]))) - 7)
            rms = float(np.sqrt(np.mean((o - r) ** 2)))
            bar = max(BF16_STEPS * ulp, 4.0 * np.sqrt(2.0) * FLOOR_FACTOR * rms)
            assert gap <= bar, (i, int(t), a, gap, bar)
            flips += 1
        logits = om.forward(oc, [int(t)])
        with orc.reversed_accumulation():
            rlogits = om.forward(rc, [int(t)])
    return flips, floor_flips, len(tokens)


def _assert_flips(name, flips, floor_flips, n):
    """The GPU's flip count against the reordered oracle's on the same
    stream: flips are coin tosses at near-ties, so the floor's count is a
    counting estimate and the slack is two standard deviations of it (at
    least one token), as in the end-to-end logits bar."""
    slack = max(1.0, 2.0 * np.sqrt(max(1, floor_flips)))
    print(f"[{name}] {n} greedy tokens: GPU took {flips} ties the other way; the reordered oracle flips "
          f"{floor_flips} on the same stream; allowed {floor_flips + slack:.1f}", flush=True)
    assert flips <= floor_flips + slack, (flips, floor_flips, slack)


def test_small_speculative_vs_oracle(gpu, orc):
    target, draft = _gpu(gpu, SMALL, 7), _gpu(gpu, SMALL, 7, layers=1)
    om = orc.Qwen3(orc.make_config(**SMALL), 7, 0.02)
    odm = orc.Qwen3(orc.make_config(**{**SMALL, "layers": 1}), 7, 0.02)
    prompt = orc.fill_tokens(14, 10, SMALL["vocab"])
    spec, _ = gpu.speculative_generate(target, target.new_cache(320), draft, draft.new_cache(320), prompt, 256,
                                       spec_k=5, eos=())
    ospec, ostats = orc.speculative_generate(om, om.new_cache(320), odm, odm.new_cache(320), prompt, 256, spec_k=5,
                                             eos=())
    print(f"oracle speculative: drafted {ostats[1]}, accepted {ostats[2]}", flush=True)
    # the oracle's own speculative output is its greedy output
    np.testing.assert_array_equal(ospec, orc.generate_greedy(om, om.new_cache(320), prompt, 256, eos=()))
    _assert_flips("SMALL vs oracle", *_agree_with_oracle_greedy(orc, om, spec, prompt, 320))


def test_4b_target_0_6b_draft_speculative(gpu, orc):
    """The Qwen3-4B-shaped target with a Qwen3-0.6B-shaped draft (config 4's
    draft; the 4B shape keeps the oracle side fast): 256 speculative tokens
    equal 256 greedy tokens exactly, and against the oracle's greedy decode
    on the same stream the GPU takes no more near-ties the other way than
    the oracle does against itself with its summation order reversed."""
    print("building 4B target + 0.6B draft", flush=True)
    target = _gpu(gpu, QWEN3_4B, 42, max_tokens=16)
    draft = _gpu(gpu, QWEN3_0_6B, 43, max_tokens=16)
    prompt = orc.fill_tokens(60, 12, QWEN3_4B["vocab"])
    greedy, _ = _spec_equals_greedy(gpu, target, draft, prompt, 256)
    om = orc.Qwen3(orc.make_config(**QWEN3_4B), 42, 0.02)
    _assert_flips("4B vs oracle", *_agree_with_oracle_greedy(orc, om, greedy, prompt, 288))


def test_32b_shape_target_0_6b_draft_speculative_loop(gpu, orc):
    """Config 4's shapes through the whole speculative loop: the
    Qwen3-32B-shaped target (2 of its 64 layers, untied head; the
    matrix-core GEMVs at M = 5) with the Qwen3-0.6B-shaped draft, both
    caches holding 2048 synthetic positions, a 6-token prompt and 64 tokens
    with 4 drafts + 1 per verify.  Speculative == greedy token for token with
    the independent draft (nothing accepted) and with a twin of the target
    as draft (everything accepted: every verify row is used), and the greedy
    tokens agree with the oracle's up to near-ties, as above."""
    print("config 4 loop: 2-layer 32B-shape target, 0.6B-shape draft, context 2048", flush=True)
    shape = dict(QWEN3_32B, layers=2)
    target = _gpu(gpu, QWEN3_32B, 13, max_tokens=16, layers=2)
    twin = _gpu(gpu, QWEN3_32B, 13, max_tokens=16, layers=2)
    draft = _gpu(gpu, QWEN3_0_6B, 14, max_tokens=16)
    prompt = orc.fill_tokens(70, 6, shape["vocab"])
    n, cap = 64, 2048 + 6 + 64 + 16

    def filled(model, seed):
        c = model.new_cache(cap)
        c.fill_synthetic(seed, 2048)
        return c

    greedy = target.generate_greedy(filled(target, 99), prompt, n, eos=())
    for d, dseed, name in ((draft, 98, "0.6B draft"), (twin, 99, "twin draft")):
        spec, stats = gpu.speculative_generate(target, filled(target, 99), d, filled(d, dseed), prompt, n, spec_k=5,
                                               eos=())
        print(f"{name}: {len(spec)} tokens, iterations {stats[0]}, drafted {stats[1]}, accepted {stats[2]}",
              flush=True)
        np.testing.assert_array_equal(spec, greedy)
    assert stats[2] == stats[1] > 0  # the twin's drafts are all accepted
    om = orc.Qwen3(orc.make_config(**shape), 13, 0.02)
    _assert_flips("32B-shape vs oracle", *_agree_with_oracle_greedy(orc, om, greedy, prompt, cap, 2048, 99))
