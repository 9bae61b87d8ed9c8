"""End-to-end parity of the GPU Qwen3 (C-ABI driver) against the CPU
oracle on identical seeded weights: logits of every position within 2e-2
relative (L2 over the vocabulary; bf16 activations / fp32 accumulation
through every layer) and greedy top-1 agreement of at least 99% over at
least 64 positions (tests/_parity.py holds the bar, and measures the
oracle's own summation-order spread beside it); cache semantics; greedy and
speculative decoding."""
import numpy as np
import pytest

from _parity import Parity
from _util import bf16_to_f32, l2_rel_err, torch_bf16_bits

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=512, inter=1536, layers=3, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)


def _pair(gpu, orc, seed=1, max_tokens=64, **kw):
    shape = {**SMALL, **kw}
    gm = gpu.Qwen3(gpu.qwen3_config(**shape), seed, 0.02, max_tokens=max_tokens)
    om = orc.Qwen3(orc.make_config(**shape), seed, 0.02)
    return gm, om


def test_weights_bit_identical(gpu, orc):
    gm, om = _pair(gpu, orc)
    for layer, slot in [(-1, 0), (0, 0), (1, 4), (2, 6)]:
        gw = gm.qlinear_numpy(layer, slot)
        ow = om.qlinear(layer, slot)
        for a, b in zip(gw, ow):
            np.testing.assert_array_equal(a, b)


def _check_logits(g, o, tol=2e-2):
    g = bf16_to_f32(torch_bf16_bits(g)).reshape(o.shape).astype(np.float64)
    o = bf16_to_f32(o).astype(np.float64)
    rows = g.reshape(-1, g.shape[-1])
    orows = o.reshape(-1, o.shape[-1])
    errs = [l2_rel_err(a, b) for a, b in zip(rows, orows)]
    agree = np.mean(np.argmax(rows, 1) == np.argmax(orows, 1))
    print(f"logits rel err (L2) max {max(errs):.2e}, top-1 agreement {agree:.3f}", flush=True)
    assert max(errs) < tol, errs
    return agree


@pytest.mark.parametrize("P", [1, 5, 8, 20, 64])
def test_prefill_logits(gpu, orc, P):
    gm, om = _pair(gpu, orc)
    toks = orc.fill_tokens(100 + P, P, SMALL["vocab"])
    gc, oc = gm.new_cache(128), om.new_cache(128)
    g = gm.forward(gc, toks, all_logits=True)
    o = om.forward(oc, toks, all_logits=True)
    _check_logits(g, o)
    assert gc.seq_len == oc.seq_len == P
    # the KV cache rows written match the oracle's
    for layer in range(SMALL["layers"]):
        for kv in (0, 1):
            ref = oc.data()[layer, kv][:, :P]
            got = gc.layer_numpy(layer, kv)[:, :P]
            assert l2_rel_err(bf16_to_f32(got), bf16_to_f32(ref)) < 2e-2, (layer, kv)


def test_prefill_and_decode_top1_over_128_positions(gpu, orc):
    """A 64-token prefill and 64 teacher-forced graph decode steps of the
    3-layer model: every position within 2e-2; top-1 agreement at least
    min(99%, the reordered oracle's own) less one position, and exact on
    every decided position (tests/_parity.py)."""
    gm, om = _pair(gpu, orc, seed=9)
    prompt = orc.fill_tokens(90, 64, SMALL["vocab"])
    gc, oc, rc = gm.new_cache(160), om.new_cache(160), om.new_cache(160)
    par = Parity("3-layer prefill 64 + decode 64")
    g = gm.forward(gc, prompt, all_logits=True)
    o = om.forward(oc, prompt, all_logits=True)
    with orc.reversed_accumulation():
        r = om.forward(rc, prompt, all_logits=True)
    par.add(torch_bf16_bits(g), o, r)
    t = int(np.argmax(bf16_to_f32(o[-1])))
    for _ in range(64):
        _, g = gm.decode_step(gc, t, want_logits=True)
        o = om.forward(oc, [t])
        with orc.reversed_accumulation():
            r = om.forward(rc, [t])
        par.add(torch_bf16_bits(g), o[None], r[None])
        t = int(np.argmax(bf16_to_f32(o)))
    err, _ = par.check()
    assert err.max() < 2e-2


def test_decode_steps_graph_vs_oracle(gpu, orc):
    """Teacher-forced decode: the graph-captured M = 1 step after a prefill."""
    gm, om = _pair(gpu, orc, seed=2)
    prompt = orc.fill_tokens(7, 12, SMALL["vocab"])
    gc, oc = gm.new_cache(64), om.new_cache(64)
    gm.forward(gc, prompt)
    om.forward(oc, prompt)
    stream = orc.fill_tokens(8, 10, SMALL["vocab"])
    for t in stream:
        nxt, g = gm.decode_step(gc, int(t), want_logits=True)
        o = om.forward(oc, [t])
        _check_logits(g, o[None])
        assert nxt == int(np.argmax(bf16_to_f32(torch_bf16_bits(g))))
    assert gc.seq_len == oc.seq_len == 22


def test_verify_width_5_after_prefill(gpu, orc):
    gm, om = _pair(gpu, orc, seed=3)
    prompt = orc.fill_tokens(9, 30, SMALL["vocab"])
    gc, oc = gm.new_cache(64), om.new_cache(64)
    gm.forward(gc, prompt)
    om.forward(oc, prompt)
    v = orc.fill_tokens(10, 5, SMALL["vocab"])
    _check_logits(gm.forward(gc, v, all_logits=True), om.forward(oc, v, all_logits=True))


def test_cache_errors_and_truncate(gpu, orc):
    gm, _ = _pair(gpu, orc, seed=4)
    c = gm.new_cache(16)
    toks = orc.fill_tokens(11, 12, SMALL["vocab"])
    gm.forward(c, toks)
    with pytest.raises(gpu.BmxError) as ei:
        gm.forward(c, toks[:5])
    assert ei.value.code == gpu.BMX_E_KV_CAPACITY and c.seq_len == 12
    with pytest.raises(gpu.BmxError):
        gm.forward(c, [SMALL["vocab"]])  # token outside the vocabulary
    a = gm.forward(c, toks[:3], all_logits=True)
    c.truncate(12)
    b = gm.forward(c, toks[:3], all_logits=True)
    np.testing.assert_array_equal(torch_bf16_bits(a), torch_bf16_bits(b))
    other = gpu.Qwen3(gpu.qwen3_config(**{**SMALL, "layers": 2}), 1, max_tokens=8)
    with pytest.raises(gpu.BmxError) as ei:
        other.forward(c, toks[:1])
    assert ei.value.code == gpu.BMX_E_SHAPE


def test_greedy_generation_teacher_forced_by_oracle(gpu, orc):
    """GPU greedy generation of 32 tokens, replayed through the oracle token
    by token: at every step the oracle's argmax is the GPU's next token,
    unless the oracle's own top-2 logits lie within 2 bf16 ulps of each
    other there (a tie that rounding alone decides)."""
    gm, om = _pair(gpu, orc, seed=5)
    prompt = orc.fill_tokens(12, 16, SMALL["vocab"])
    g = gm.generate_greedy(gm.new_cache(128), prompt, 32, eos=())
    assert len(g) == 32
    oc = om.new_cache(128)
    logits = om.forward(oc, prompt)
    ties = 0
    for i, t in enumerate(g):
        o = bf16_to_f32(logits).astype(np.float64)
        top = np.argsort(o)[-2:]
        if int(np.argmax(o)) != int(t):
            gap = o[top[1]] - o[top[0]]
            assert gap <= 2 * abs(o[top[1]]) * 2.0 ** -7, (i, int(t), int(np.argmax(o)), gap)
            ties += 1
        logits = om.forward(oc, [int(t)])
    assert ties <= 1, ties


def test_greedy_stops_at_eos(gpu, orc):
    gm, _ = _pair(gpu, orc, seed=6)
    prompt = orc.fill_tokens(13, 8, SMALL["vocab"])
    g = gm.generate_greedy(gm.new_cache(64), prompt, 12, eos=())
    stop = int(g[3])
    g2 = gm.generate_greedy(gm.new_cache(64), prompt, 12, eos=(stop,))
    first = int(np.argmax(g == stop))
    np.testing.assert_array_equal(g2, g[:first])


def test_decode_greedy_queued_steps_equal_single_steps(gpu, orc):
    """bmx_decode_greedy queues graph replays ahead of the token it checks,
    each replay taking its token and position from the previous one on the
    device.  Its tokens, the cache length and the K/V rows it leaves equal
    those of bmx_qwen3_decode_step one token at a time; an eos token met with
    replays queued past it rewinds the cache to the steps the loop took, and
    the next loop overwrites those rows; a cache that fills up mid-loop ends
    with the capacity error and the tokens decoded before it."""
    gm, _ = _pair(gpu, orc, seed=8)
    prompt = orc.fill_tokens(14, 10, SMALL["vocab"])
    n = 40
    ref_c = gm.new_cache(64)
    tok = int(gm.forward(ref_c, prompt).float().argmax())
    ref = [tok]
    for _ in range(n - 1):
        ref.append(gm.decode_step(ref_c, ref[-1]))
    c = gm.new_cache(64)
    assert int(gm.forward(c, prompt).float().argmax()) == tok
    got = gm.decode_greedy(c, tok, n, eos=())
    np.testing.assert_array_equal(got, ref)
    assert c.seq_len == ref_c.seq_len == len(prompt) + n - 1
    for layer in range(SMALL["layers"]):
        for kv in (0, 1):
            np.testing.assert_array_equal(c.layer_numpy(layer, kv)[:, : c.seq_len],
                                          ref_c.layer_numpy(layer, kv)[:, : c.seq_len])
    # eos at a token's first occurrence, the third token or later where the
    # greedy sequence has one: `k` emitted and `k` steps kept; replays
    # queued past the eos wrote rows the rewind drops, and continuing
    # rewrites them
    first = [i for i in range(1, n) if ref[i] not in ref[:i]]
    assert first, ref  # a fixed point from the first token on
    k = next((i for i in first if i >= 3), first[0])
    print(f"greedy tokens {ref}; eos at {k}", flush=True)
    c.truncate(len(prompt))
    got = gm.decode_greedy(c, tok, n, eos=(ref[k],))
    np.testing.assert_array_equal(got, ref[:k])
    assert c.seq_len == len(prompt) + k
    rest = gm.decode_greedy(c, ref[k], n - k, eos=())
    np.testing.assert_array_equal(rest, ref[k:])
    assert c.seq_len == ref_c.seq_len
    # room for 6 more positions: 7 tokens, then the capacity error
    small = gm.new_cache(len(prompt) + 6)
    gm.forward(small, prompt)
    with pytest.raises(gpu.BmxError) as ei:
        gm.decode_greedy(small, tok, n, eos=())
    assert ei.value.code == gpu.BMX_E_KV_CAPACITY
    np.testing.assert_array_equal(ei.value.tokens, ref[:7])
    assert small.seq_len == len(prompt) + 6


def test_long_context_decode_and_verify(gpu, orc):
    """Long contexts after identical synthetic KV fills of GPU and oracle
    caches: a graph decode step at position 65535, the last one the 256 key
    splits of 256 of the model's attention workspace cover; and at context
    20000 a 5-token and a 16-token verify (fused split-key attention over 79
    splits) and a 24-token forward (96 query rows per kv head, past the
    split-key path's 64, so flash attention at that offset).  Logits against
    the oracle and its reordered floor."""
    gm, om = _pair(gpu, orc, seed=12, max_tokens=24)
    for ctx, cap, widths in [(65535, 65536, [1]), (20000, 20480, [5, 16, 24])]:
        print(f"context {ctx}: synthetic KV fills", flush=True)
        gc, oc, rc = gm.new_cache(cap), om.new_cache(cap), om.new_cache(cap)
        for c in (gc, oc, rc):
            c.fill_synthetic(77, ctx)
        np.testing.assert_array_equal(gc.layer_numpy(2, 1)[:, :ctx], oc.data()[2, 1][:, :ctx])
        par = Parity(f"SMALL at context {ctx}")
        for i, M in enumerate(widths):
            toks = orc.fill_tokens(300 + i, M, SMALL["vocab"])
            if M == 1:
                g = gm.decode_step(gc, int(toks[0]), want_logits=True)[1][None]
            else:
                g = gm.forward(gc, toks, all_logits=True)
            o = om.forward(oc, toks, all_logits=True)
            with orc.reversed_accumulation():
                r = om.forward(rc, toks, all_logits=True)
            par.add(torch_bf16_bits(g), o, r)
            assert gc.seq_len == oc.seq_len == ctx + M
            for c in (gc, oc, rc):
                c.truncate(ctx)
        par.check()
        del gc, oc, rc


def test_prefill_unsplit_fused_epilogues(gpu, orc):
    """A 2048-token prefill through one Qwen3-4B-shaped layer: at this size
    the o and down GEMMs run unsplit with the residual add in their epilogue,
    gate|up runs as one GEMM with the SwiGLU epilogue (the smaller prefills
    above split K and add the residual in the reduction), and the q|k|v GEMM
    norms and rotates q and k and writes the cache rows in its epilogue;
    logits of every position and the cache rows against the oracle."""
    shape = dict(hidden=2560, inter=9728, layers=1, n_heads=32, n_kv_heads=8, head_dim=128, vocab=1024)
    gm = gpu.Qwen3(gpu.qwen3_config(**shape), 5, 0.02, max_tokens=2048)
    om = orc.Qwen3(orc.make_config(**shape), 5, 0.02)
    toks = orc.fill_tokens(21, 2048, shape["vocab"])
    gc, oc = gm.new_cache(2100), om.new_cache(2100)
    g = gm.forward(gc, toks, all_logits=True)
    print("oracle forward (2048 tokens)", flush=True)
    o = om.forward(oc, toks, all_logits=True)
    assert _check_logits(g, o) >= 0.9
    for kv in (0, 1):
        ref = oc.data()[0, kv][:, :2048]
        got = gc.layer_numpy(0, kv)[:, :2048]
        assert l2_rel_err(bf16_to_f32(got), bf16_to_f32(ref)) < 2e-2, kv
        # rows past the prefill are not written
        assert not gc.layer_numpy(0, kv)[:, 2048:].any(), kv


def _write_projection(gpu, gm, layer, slot, arrays):
    """Writes host arrays (w, s, b) into a projection of the GPU model
    through the device pointers bmx_qwen3_qlinear hands out."""
    import ctypes

    ptrs = [ctypes.c_void_p() for _ in range(3)]
    N, K = ctypes.c_int(), ctypes.c_int()
    gpu.call("bmx_qwen3_qlinear", gm.h, layer, slot, *[ctypes.byref(q) for q in ptrs], ctypes.byref(N),
             ctypes.byref(K))
    for dst, src in zip(ptrs, arrays):
        src = np.ascontiguousarray(src)
        assert gpu._hip().hipMemcpy(dst, src.ctypes.data_as(ctypes.c_void_p), src.nbytes, 1) == 0


def test_prefill_reads_weights_written_through_qlinear(gpu, orc):
    """The prefill GEMMs read a group-major copy of each layer projection;
    a projection written through the pointers of bmx_qwen3_qlinear is seen
    by the next prefill: with layer 1's gate and down and layer 0's v
    projection replaced in both models the logits follow the oracle's, and
    with the old weights written back they are the first prefill's bit for
    bit."""
    gm, om = _pair(gpu, orc)
    toks = orc.fill_tokens(77, 40, SMALL["vocab"])
    g0 = torch_bf16_bits(gm.forward(gm.new_cache(64), toks, all_logits=True))
    old = {key: [a.copy() for a in gm.qlinear_numpy(*key)] for key in [(1, 4), (1, 6), (0, 2)]}
    for (layer, slot), seed in [((1, 4), 5), ((1, 6), 7), ((0, 2), 6)]:
        w, s, b = old[(layer, slot)]
        rng = np.random.default_rng(seed)
        new = (rng.integers(0, 2**32, w.shape, dtype=np.uint32), s[::-1].copy(), b[:, ::-1].copy())
        _write_projection(gpu, gm, layer, slot, new)
        for dst, src in zip(om.qlinear(layer, slot), new):
            dst[...] = src
    g1 = gm.forward(gm.new_cache(64), toks, all_logits=True)
    o1 = om.forward(om.new_cache(64), toks, all_logits=True)
    _check_logits(g1, o1)
    assert not np.array_equal(torch_bf16_bits(g1), g0)
    for key, arrays in old.items():
        _write_projection(gpu, gm, *key, arrays)
    g2 = torch_bf16_bits(gm.forward(gm.new_cache(64), toks, all_logits=True))
    np.testing.assert_array_equal(g2, g0)


def test_qwen3_4b_shape_prefill_and_decode(gpu, orc):
    """Full Qwen3-4B shape (36 layers, 151936 vocab) at short context: a
    9-token prefill, 32 teacher-forced decode steps and an 8-token verify
    forward (the M = 8 GEMV path with the fused norm), 49 positions against
    the oracle and the oracle's own summation-order spread
    (tests/_parity.py)."""
    shape = dict(hidden=2560, inter=9728, layers=36, n_heads=32, n_kv_heads=8, head_dim=128, vocab=151936)
    print("building 4B models", flush=True)
    gm = gpu.Qwen3(gpu.qwen3_config(**shape), 42, 0.02, max_tokens=16)
    om = orc.Qwen3(orc.make_config(**shape), 42, 0.02)
    print("built", flush=True)
    prompt = orc.fill_tokens(15, 9, shape["vocab"])
    gc, oc, rc = gm.new_cache(64), om.new_cache(64), om.new_cache(64)
    par = Parity("4B shape, short context")

    def both(toks):
        g = gm.forward(gc, toks, all_logits=True)
        o = om.forward(oc, toks, all_logits=True)
        with orc.reversed_accumulation():
            r = om.forward(rc, toks, all_logits=True)
        par.add(torch_bf16_bits(g), o, r)
        return o

    o = both(prompt)
    t = int(np.argmax(bf16_to_f32(o[-1])))
    for _ in range(32):
        _, g = gm.decode_step(gc, t, want_logits=True)
        o = om.forward(oc, [t])
        with orc.reversed_accumulation():
            r = om.forward(rc, [t])
        par.add(torch_bf16_bits(g), o[None], r[None])
        t = int(np.argmax(bf16_to_f32(o)))
    both(orc.fill_tokens(17, 8, shape["vocab"]))
    par.check()
    print("done", flush=True)


def test_two_models_concurrent_prefill(gpu, orc):
    """Two models' prefills (split-K GEMMs) launched back to back on their own
    streams, no sync in between: each matches its oracle (no shared scratch)."""
    import torch

    toks = orc.fill_tokens(5, 9, SMALL["vocab"])
    pairs = [_pair(gpu, orc, seed=s, max_tokens=32) for s in (31, 32)]
    caches = [gm.new_cache(64) for gm, _ in pairs]
    outs = [gm.forward(c, toks, all_logits=True) for (gm, _), c in zip(pairs, caches)]
    torch.cuda.synchronize()
    for (gm, om), g in zip(pairs, outs):
        o = om.forward(om.new_cache(64), toks, all_logits=True)
        assert _check_logits(g, o) >= 0.9


def test_qmatmul_two_streams(gpu, orc):
    """The public GEMM path (M > 8, split K) on two streams at once."""
    import torch

    from _util import to_torch_bf16

    M, N, K = 64, 1024, 2560
    args = []
    for i in range(2):
        wq, s, b = orc.init_qlinear(40 + i, N, K)
        x = orc.fill_normal_bf16(50 + i, M * K).reshape(M, K)
        w_d, s_d, b_d = gpu.init_qlinear(40 + i, N, K)
        args.append((to_torch_bf16(x), w_d, s_d, b_d, orc.qlinear(x, wq, s, b)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for (x, w, s, b, _), st in zip(args, streams):
        with torch.cuda.stream(st):
            outs.append(gpu.quantized_matmul(x, w, s, b))
    torch.cuda.synchronize()
    for (_, _, _, _, ref), y in zip(args, outs):
        yb = bf16_to_f32(torch_bf16_bits(y)).astype(np.float64)
        r = bf16_to_f32(ref).astype(np.float64)
        assert np.mean(np.abs(yb - r) <= np.maximum(2 * np.abs(r) * 2.0 ** -7, 1e-3 * np.max(np.abs(r)))) > 0.999
