"""Benchmark: Qwen3-4B-shaped 4-bit decode at batch 1 on one MI355X, plus the
qmv sweep over the Qwen3-4B projection shapes.

Workload (the headline `value`): a random-init Qwen3-4B-shaped model
(hidden 2560, intermediate 9728, 36 layers, 32 q / 8 kv heads, head_dim 128,
vocab 151936, MLX 4-bit gs64), KV cache [36, 2, 8, 4352, 128] bf16, a
4096-token seeded random prompt prefilled untimed, then greedy decode.  One
step = one decode token: a graph launch of the whole forward (36 layers +
lm_head + argmax), run by the library's greedy decode loop, which checks each
token for eos on the host as the reference's generate loop does while the
next steps are already queued on the GPU.  `value` = decode tokens / s.
`config.decode_step_sync_tok_s` times the same tokens one synchronous decode
step at a time (token read back before the next launch).

`roofline`: the decode step's dominant kernel -- the fused decode attention
(QK-norm, RoPE, KV-row write, split-key GQA attention and merge; one launch
per layer, the largest share of a decode token) -- for one new token at
position 4096, launched through its C-ABI entry point (the kernel the decode
graph launches) in a graph over 36 distinct layer caches (604 MB of K/V:
more than the 256 MB Infinity Cache), timed with HIP events on the capturing
stream; algorithmic bytes per launch = K and V rows of the 4096 cached
positions plus the new token's rows, the q row, the norm weights and the
output.  `step_roofline`: the whole decode step, bytes every token must read
(weights + the K/V of the context) over the measured time per token.
`config.qmv_sweep`: the M = 1 GEMV per Qwen3-4B projection shape, 1000
launches per shape in a graph rotating over >= 1 GiB of distinct weights.

`cpu_baseline`: the C restatement of the same decode step (oracle/, OpenMP)
on this host's cores, timed over a bounded sample of decode tokens at context
4096 (KV positions filled synthetically instead of a CPU prefill), with the
host's CPU model, the threads used and a STREAM-triad bandwidth beside it.

The other configurations run in the default invocation too and are reported
under `config`: the qmm sweep (M = 5, 128, 512, 2048 over the eleven
Qwen3-4B / 8B projection shapes), greedy speculative decoding with a
Qwen3-32B-shaped target and a Qwen3-0.6B-shaped draft, and the
Qwen3-0.6B-shaped prompt-32 / 64-token greedy run on the GPU and, beside it,
on the host cores through the oracle.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "base-mlx_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
SHAPE_4B = dict(hidden=2560, inter=9728, layers=36, n_heads=32, n_kv_heads=8, head_dim=128, vocab=151936)
QMV_SHAPES = [(4096, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (2560, 9728), (151936, 2560)]
ROOF_SHAPE = (9728, 2560)
QMM_SHAPES = QMV_SHAPES + [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (151936, 4096)]
QMM_M = [5, 128, 512, 2048]
MFMA_BF16_PEAK_TFLOPS = 2500.0
PREFILLS = 5  # warm prefills timed for the median


def _profile_value(name, key):
    """A `key: value` line of a committed profiles/ summary; None if absent."""
    try:
        for line in open(os.path.join(ROOT, "profiles", name)):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1].split()[0])
    except (OSError, ValueError, IndexError):
        pass
    return None


TRAFFIC_PROFILE = "decode_attention_ctx4096_pmc.md"
TRACE_PROFILE = "decode_attention_ctx4096_pmc.md"


def measured_traffic():
    """HBM bytes per launch of the roofline kernel, read from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE scaled by a copy of
    known size; not measured in this run); None when it is absent."""
    v = _profile_value(TRAFFIC_PROFILE, "traffic_bytes_per_launch")
    return None if v is None else int(v)


def traced_duration_us():
    """Average duration of the roofline kernel in the committed rocprofv3
    kernel trace of the counter workload (`--profile-roofline`: the same
    launch at position 4096 over 36 layer caches; the tracer's per-dispatch
    timestamps, not measured in this run, whose `achieved` uses HIP events
    around graph replays); None when that summary is absent."""
    return _profile_value(TRACE_PROFILE, "roofline_kernel_trace_avg_us")


def host_info():
    """CPU model, logical CPUs in this process's affinity mask, OpenMP
    threads of the oracle, and a STREAM-triad bandwidth of the host."""
    import oracle

    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "affinity_cpus": len(os.sched_getaffinity(0)), "threads": oracle.num_threads(),
            "stream_triad_GBps": round(oracle.stream_triad_gbs(), 1)}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def qmv_bytes(N, K, M=1):
    return int(0.5625 * N * K + 2 * M * K + 2 * M * N)


def time_qmv(bmx, torch, N, K, reps=1000, M=1):
    """Average duration (us) of one qmv launch over `reps` timed launches
    (one graph replay, after an untimed one), rotating over >= 1 GiB of
    distinct weights; HIP events on the capturing stream."""
    nbytes = qmv_bytes(N, K, M)
    copies = max(2, -(-(1 << 30) // nbytes))
    ws = [bmx.init_qlinear(5000 + i, N, K) for i in range(copies)]
    x = bmx.fill_normal_bf16(77, (M, K))
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    reps = max(reps, copies)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        for i in range(4):
            bmx.quantized_matmul(x, *ws[i % copies], out=y)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            for i in range(reps):
                bmx.quantized_matmul(x, *ws[i % copies], out=y)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    del g, ws
    torch.cuda.empty_cache()
    return us, nbytes


ATT_CTX = 4096  # cached positions before the first timed decode token
ATT_LAYERS = 36


def attention_bytes(ctx, Hq=32, Hkv=8, D=128):
    """Algorithmic bytes of one decode-attention launch for the token at
    position ctx: K and V rows of the ctx cached positions, the q, k and v
    rows of the new token, its K / V rows written to the cache, the two norm
    weights and the output row (bf16)."""
    return 2 * 2 * ctx * Hkv * D + 2 * Hq * D + 2 * 2 * Hkv * D + 2 * 2 * Hkv * D + 2 * 2 * D + 2 * Hq * D


def _attention_inputs(bmx, torch, ctx, layers, cap=4352, Hq=32, Hkv=8):
    kcs = [bmx.fill_normal_bf16(100 + i, (Hkv, cap, 128)) for i in range(layers)]
    vcs = [bmx.fill_normal_bf16(200 + i, (Hkv, cap, 128)) for i in range(layers)]
    q = bmx.fill_normal_bf16(1, (1, Hq * 128))
    k = bmx.fill_normal_bf16(2, (1, Hkv * 128))
    v = bmx.fill_normal_bf16(3, (1, Hkv * 128))
    qn = bmx.fill_normal_bf16(4, (128,))
    kn = bmx.fill_normal_bf16(5, (128,))
    return kcs, vcs, q, k, v, qn, kn


def time_decode_attention(bmx, torch, ctx=ATT_CTX, layers=ATT_LAYERS, per_layer=28):
    """Average duration (us) of the decode step's attention launch
    (bmx_qk_norm_rope_kv_attention: the kernel the decode graph launches per
    layer) for one token at position ctx, Qwen3-4B head layout: a graph of
    layers x per_layer launches cycling over `layers` distinct layer caches
    (each launch reads K / V no other launch near it read), HIP events on
    the capturing stream around one replay after an untimed one."""
    kcs, vcs, q, k, v, qn, kn = _attention_inputs(bmx, torch, ctx, layers)
    ws = bmx.attention_workspace(32, 1)
    reps = layers * per_layer
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        for i in range(layers):
            bmx.qk_norm_rope_kv_attention(q, k, v, qn, kn, kcs[i], vcs[i], ctx, workspace=ws, stream=st)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            for i in range(reps):
                bmx.qk_norm_rope_kv_attention(q, k, v, qn, kn, kcs[i % layers], vcs[i % layers], ctx, workspace=ws,
                                              stream=st)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    del g, kcs, vcs
    torch.cuda.empty_cache()
    return us, attention_bytes(ctx)


def decode_weight_bytes(shape):
    """Packed weight bytes one decode token reads: every projection of every
    layer and the (tied) vocabulary head, 0.5625 B per weight, plus the norm
    weights."""
    H, I, L = shape["hidden"], shape["inter"], shape["layers"]
    qd, kvd = shape["n_heads"] * shape["head_dim"], shape["n_kv_heads"] * shape["head_dim"]
    per_layer = qd * H + 2 * kvd * H + H * qd + 2 * I * H + H * I
    norms = L * (2 * H + 2 * shape["head_dim"]) * 2 + 2 * H
    return int(0.5625 * (L * per_layer + shape["vocab"] * H)) + norms


def time_qmm(bmx, torch, M, N, K):
    """Average duration (us) of one quantized matmul of M rows, graph-captured,
    rotating over >= 1 GiB of distinct weights (at least 2 copies)."""
    nbytes = qmv_bytes(N, K, M)
    copies = max(2, -(-(1 << 30) // int(0.5625 * N * K)))
    flops = 2.0 * M * N * K
    reps = max(copies, min(200, int(2e12 / flops) + 2))
    ws = [bmx.init_qlinear(6000 + i, N, K) for i in range(copies)]
    x = bmx.fill_normal_bf16(78, (M, K))
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        bmx.quantized_matmul(x, *ws[0], out=y)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            for i in range(reps):
                bmx.quantized_matmul(x, *ws[i % copies], out=y)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    del g, ws
    torch.cuda.empty_cache()
    return us, nbytes, flops


# Qwen3-30B-A3B-shaped routed experts: 128 experts, top-8, hidden 2048,
# moe_intermediate 768 (gate|up concatenated: N = 1536)
MOE_SHAPES = [("gate_up", 1536, 2048, 8), ("down", 2048, 768, 1)]


def time_gather(bmx, torch, N, K, x_bcast, E=128, top_k=8, reps=200):
    """Average duration (us) of one routed decode projection (one token, top_k
    routes to distinct experts), graph-captured over rotating route sets; the
    128 experts of each of 4 stacked copies (>= 1 GiB in all) keep the reads
    HBM-cold."""
    import numpy as np

    per_expert = int(0.5625 * N * K)
    copies = max(1, -(-(1 << 30) // (E * per_expert)))
    ws = []
    for c in range(copies):
        ex = [bmx.init_qlinear(9000 + c * E + e, N, K) for e in range(E)]
        ws.append(tuple(torch.stack([t[i] for t in ex]).contiguous() for i in range(3)))
        del ex
    rng = np.random.default_rng(5)
    routes = [torch.from_numpy(rng.choice(E, top_k, replace=False).astype(np.int32)).cuda() for _ in range(reps)]
    x = bmx.fill_normal_bf16(79, (top_k // x_bcast, 1, K))
    y = torch.empty(top_k, 1, N, dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        bmx.gather_qmm(x, *ws[0], routes[0], x_bcast, out=y)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            for i in range(reps):
                bmx.gather_qmm(x, *ws[i % copies], routes[i], x_bcast, out=y)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    nbytes = top_k * per_expert + 2 * (top_k // x_bcast) * K + 2 * top_k * N
    del g, ws
    torch.cuda.empty_cache()
    return us, nbytes


def moe_bench(bmx, torch):
    out = []
    for name, N, K, xb in MOE_SHAPES:
        us, nb = time_gather(bmx, torch, N, K, xb)
        gbs = nb / us / 1e3
        out.append({"proj": name, "experts": 128, "top_k": 8, "N": N, "K": K, "us": round(us, 3),
                    "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"gather_qmm {name} 8 of 128 experts ({N}, {K}): {us:.2f} us, {gbs:.0f} GB/s")
    return out


def qmm_sweep(bmx, torch):
    out = []
    for M in QMM_M:
        for (N, K) in QMM_SHAPES:
            us, nb, fl = time_qmm(bmx, torch, M, N, K)
            tf = fl / us / 1e6
            out.append({"M": M, "N": N, "K": K, "us": round(us, 2), "TFLOP/s": round(tf, 1),
                        "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "GB/s": round(nb / us / 1e3, 1)})
            log(f"qmm M={M} N={N} K={K}: {us:.1f} us, {tf:.1f} TFLOP/s ({100 * tf / MFMA_BF16_PEAK_TFLOPS:.1f}% of "
                f"2.5 PF bf16), {nb / us / 1e3:.0f} GB/s")
    return out


def speculative_bench(bmx, torch, new_tokens=512, prompt_len=2048, spec_k=5):
    """Greedy speculative decoding: a Qwen3-32B-shaped 4-bit target (64 layers,
    untied head) verifying 4 drafted tokens + 1 per step (M = 5) from a
    Qwen3-0.6B-shaped draft, after a seeded prompt.  With independent random
    models almost no draft is accepted, so this measures the verify-step cost.
    Returns accepted tokens/s of the generation phase, the verify-step and
    draft-step costs and the acceptance counts."""
    import numpy as np

    t0 = time.time()
    target = bmx.Qwen3(bmx.qwen3_config(**bmx.QWEN3_32B), 42, 0.02, max_tokens=prompt_len)
    draft = bmx.Qwen3(bmx.qwen3_config(**bmx.QWEN3_0_6B), 43, 0.02, max_tokens=prompt_len)
    cap = prompt_len + new_tokens + 2 * spec_k + 8
    tc, dc = target.new_cache(cap), draft.new_cache(cap)
    prompt = np.array([int(v) for v in np.random.default_rng(13).integers(0, 151936, prompt_len)], np.uint32)
    torch.cuda.synchronize()
    log(f"speculative: 32B target + 0.6B draft ready in {time.time() - t0:.1f}s")
    # prefill cost alone (both models), then reset
    t0 = time.perf_counter()
    target.forward(tc, prompt)
    draft.forward(dc, prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    tc.reset()
    dc.reset()
    t0 = time.perf_counter()
    toks, stats = bmx.speculative_generate(target, tc, draft, dc, prompt, new_tokens, spec_k=spec_k, eos=())
    torch.cuda.synchronize()
    total_s = time.perf_counter() - t0
    gen_s = max(total_s - prefill_s, 1e-9)
    # verify step: one M = 5 target forward at the final context, rewound
    seq = tc.seq_len
    v = np.array(toks[:spec_k], np.uint32)
    target.forward(tc, v)
    tc.truncate(seq)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        target.forward(tc, v)
        tc.truncate(seq)
    torch.cuda.synchronize()
    verify_ms = (time.perf_counter() - t0) * 100.0
    res = {"accepted_tokens_per_s": round(len(toks) / gen_s, 2), "tokens": int(len(toks)),
           "iterations": int(stats[0]), "drafted": int(stats[1]), "accepted": int(stats[2]),
           "verify_step_ms": round(verify_ms, 3), "prefill_ms_both_models": round(prefill_s * 1000, 1),
           "wall_s": round(total_s, 2), "prompt_tokens": prompt_len, "spec_k": spec_k,
           "workload": "Qwen3-32B-shape 4-bit target + Qwen3-0.6B-shape draft, greedy speculative, batch 1"}
    log(f"speculative: {res}")
    target.close()
    draft.close()
    del tc, dc
    torch.cuda.empty_cache()
    return res


def small_model_bench(bmx, torch, prompt_len=32, new_tokens=64, seed=7, cpu=True):
    """The Qwen3-0.6B-shaped model (28 layers, hidden 1024, tied head): a
    32-token seeded prompt, then 64 greedy decode tokens -- on the GPU
    (prefill forward, then the greedy decode loop of graph replays) and, as the reference
    runs this configuration on its CPU path, with the oracle on the host
    cores (prefill forward, then one forward per token).  Also reports how
    many leading greedy tokens the two agree on (random-init logits have
    near-ties, where fp32 summation order alone can flip a token)."""
    import numpy as np

    shape = dict(bmx.QWEN3_0_6B, head_dim=128, vocab=151936)
    prompt = np.array([int(v) for v in np.random.default_rng(seed).integers(0, 151936, prompt_len)], np.uint32)
    m = bmx.Qwen3(bmx.qwen3_config(**shape), seed, 0.02, max_tokens=prompt_len)
    c = m.new_cache(prompt_len + new_tokens + 8)
    m.forward(c, prompt)  # first use: one-time setup
    c.reset()
    for _ in range(4):  # captures the decode graph
        m.decode_step(c, 1)
    c.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = m.forward(c, prompt)
    tok = int(torch.argmax(logits.float()).item())
    torch.cuda.synchronize()
    gpu_prefill = time.perf_counter() - t0
    t0 = time.perf_counter()
    gpu_toks = [int(v) for v in m.decode_greedy(c, tok, new_tokens, eos=())]
    torch.cuda.synchronize()
    gpu_decode = time.perf_counter() - t0
    m.close()
    del c
    res = {"workload": "Qwen3-0.6B-shape 4-bit, 32-token prompt, 64 greedy tokens, batch 1",
           "gpu_prefill_ms": round(gpu_prefill * 1000, 2),
           "gpu_decode_tok_s": round((new_tokens - 1) / gpu_decode, 1)}
    if cpu:
        import oracle

        om = oracle.Qwen3(oracle.make_config(**shape), seed, 0.02)
        oc = om.new_cache(prompt_len + new_tokens + 8)
        t0 = time.perf_counter()
        ol = om.forward(oc, prompt)
        cpu_prefill = time.perf_counter() - t0
        t = int(np.argmax(oracle.bf16_to_f32(ol)))
        cpu_toks = [t]
        t0 = time.perf_counter()
        for _ in range(new_tokens - 1):
            t = int(np.argmax(oracle.bf16_to_f32(om.forward(oc, np.array([t], np.uint32)))))
            cpu_toks.append(t)
        cpu_decode = time.perf_counter() - t0
        om.close()
        agree = 0
        while agree < new_tokens and gpu_toks[agree] == cpu_toks[agree]:
            agree += 1
        res.update({"cpu_prefill_ms": round(cpu_prefill * 1000, 1),
                    "cpu_decode_tok_s": round((new_tokens - 1) / cpu_decode, 2),
                    "cpu_threads": oracle.num_threads(), "cpu_kind": "port (oracle/, OpenMP)",
                    "greedy_tokens_agreeing": agree})
    log(f"0.6B shape: {res}")
    torch.cuda.empty_cache()
    return res


def profile_roofline(bmx, torch, launches=200):
    """Counter-collection workload: the roofline kernel (the decode step's
    attention launch at position 4096) launched eagerly over 36 layer
    caches, the gate/up-shape GEMV (rotating over >= 1 GiB of weights), then
    a plain 256 MiB device copy as the calibration kernel whose FETCH_SIZE /
    WRITE_SIZE must read 256 MiB."""
    kcs, vcs, q, k, v, qn, kn = _attention_inputs(bmx, torch, ATT_CTX, ATT_LAYERS)
    aws = bmx.attention_workspace(32, 1)
    for i in range(launches):
        bmx.qk_norm_rope_kv_attention(q, k, v, qn, kn, kcs[i % ATT_LAYERS], vcs[i % ATT_LAYERS], ATT_CTX,
                                      workspace=aws)
    torch.cuda.synchronize()
    del kcs, vcs
    N, K = ROOF_SHAPE
    nbytes = qmv_bytes(N, K)
    copies = max(2, -(-(1 << 30) // nbytes))
    ws = [bmx.init_qlinear(5000 + i, N, K) for i in range(copies)]
    x = bmx.fill_normal_bf16(77, (1, K))
    y = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
    for i in range(launches):
        bmx.quantized_matmul(x, *ws[i % copies], out=y)
    torch.cuda.synchronize()
    del ws
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile-roofline: {launches} decode attention launches at position {ATT_CTX} "
        f"({attention_bytes(ATT_CTX)} algorithmic bytes each), {launches} qmv launches N={N} K={K} "
        f"({nbytes} algorithmic bytes each), 10 copies of {256 << 20} bytes")


def profile_mfma(bmx, torch, launches=20):
    """Counter-collection workload for the matrix-core kernels: the GEMM at
    M = 2048 on the 4B gate/up (9728 x 2560) and 8B (12288 x 4096) shapes,
    and causal prefill attention over 4096 tokens at the Qwen3-4B head layout
    (32 q / 8 kv heads, head_dim 128), each launched `launches` times."""
    for (N, K) in [(9728, 2560), (12288, 4096)]:
        w, s, b = bmx.init_qlinear(7, N, K)
        x = bmx.fill_normal_bf16(8, (2048, K))
        y = torch.empty(2048, N, dtype=torch.bfloat16, device="cuda")
        for _ in range(launches):
            bmx.quantized_matmul(x, w, s, b, out=y)
        torch.cuda.synchronize()
        log(f"profile-mfma: {launches} GEMMs M=2048 N={N} K={K} ({2 * 2048 * N * K:.3e} flop each)")
    T = 4096
    q = bmx.fill_normal_bf16(9, (32, T, 128))
    k = bmx.fill_normal_bf16(10, (8, T, 128))
    v = bmx.fill_normal_bf16(11, (8, T, 128))
    for _ in range(launches):
        bmx.attention(q, k, v, 0, use_workspace=False)
    torch.cuda.synchronize()
    log(f"profile-mfma: {launches} causal prefill attentions, 4096 tokens, 32 q / 8 kv heads")


def profile_bf16_gemm(torch, launches=50):
    """Reference figures for the prefill GEMMs: torch.matmul (hipBLASLt) on bf16
    operands of the Qwen3-4B 4096-token prefill shapes (x [4096, K] times a
    bf16 W^T [K, N]), timed with HIP events over `launches` back-to-back calls."""
    for name, (N, K) in [("q|k|v", (6144, 2560)), ("o", (2560, 4096)), ("gate|up", (19456, 2560)),
                         ("down", (2560, 9728))]:
        x = torch.randn(4096, K, device="cuda", dtype=torch.bfloat16)
        w = torch.randn(N, K, device="cuda", dtype=torch.bfloat16)
        for _ in range(5):
            y = x @ w.t()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(launches):
            y = x @ w.t()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / launches
        log(f"bf16 GEMM ({name}) 4096 x {N} x {K}: {us:.1f} us, {2 * 4096 * N * K / us / 1e6:.0f} TFLOP/s")
        del x, w, y


def cpu_baseline(tokens, ctx=4096, seed=42):
    """Oracle decode of `tokens` tokens at context `ctx` on the host cores."""
    import numpy as np

    import oracle

    cfg = oracle.make_config(**SHAPE_4B)
    t0 = time.time()
    m = oracle.Qwen3(cfg, seed, 0.02)
    cache = m.new_cache(ctx + tokens + 1)
    cache.fill_synthetic(1234, ctx)
    log(f"cpu baseline: model + cache ready in {time.time() - t0:.1f}s")
    tok = np.array([1], np.uint32)
    m.forward(cache, tok)  # first step untimed (page-in)
    t0 = time.time()
    for _ in range(tokens):
        logits = m.forward(cache, tok)
        tok = np.array([int(np.argmax(oracle.bf16_to_f32(logits)))], np.uint32)
    dt = time.time() - t0
    m.close()
    return tokens / dt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode tokens (rewound afterwards)")
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--cpu-tokens", type=int, default=8, help="decode tokens in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the qmv sweep")
    ap.add_argument("--no-qmm-sweep", action="store_true",
                    help="skip the quantized GEMM sweep at M = 5, 128, 512, 2048 (4B and 8B projection shapes)")
    ap.add_argument("--no-speculative", action="store_true",
                    help="skip 32B-target / 0.6B-draft greedy speculative decoding (M = 5 verify)")
    ap.add_argument("--no-small", action="store_true",
                    help="skip the Qwen3-0.6B-shape prompt-32 / 64-token decode (GPU and oracle on the host)")
    ap.add_argument("--moe", action="store_true",
                    help="also time gather_qmm on Qwen3-30B-A3B-shaped routed experts (decode, top-8 of 128)")
    ap.add_argument("--profile-roofline", action="store_true",
                    help="only run the roofline GEMV and a copy of known size (for rocprofv3 --pmc)")
    ap.add_argument("--profile-mfma", action="store_true",
                    help="only run the M = 2048 GEMMs and a 4096-token prefill attention (for rocprofv3 --pmc)")
    ap.add_argument("--profile-bf16-gemm", action="store_true",
                    help="only time torch.matmul (hipBLASLt) on bf16 operands of the 4096-token prefill GEMM shapes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs on one GPU: this build has no multi-GPU path (see DESIGN.md, sharding)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import bmx

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.profile_roofline:
        profile_roofline(bmx, torch)
        return
    if args.profile_mfma:
        profile_mfma(bmx, torch)
        return
    if args.profile_bf16_gemm:
        profile_bf16_gemm(torch)
        return
    cap = args.prompt + max(args.steps, args.warmup)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        log("building Qwen3-4B-shaped model")
        model = bmx.Qwen3(bmx.qwen3_config(**SHAPE_4B), 42, 0.02, max_tokens=min(args.prompt, 4096))
        cache = model.new_cache(max(cap, 4352))
        prompt = np.array([int(v) for v in np.random.default_rng(11).integers(0, 151936, args.prompt)], np.uint32)
        # prefill: the first forward of the process also pays one-time setup
        # (LDS limits, the split-K buffer); then PREFILLS warm ones, each
        # timed with HIP events on the stream (tokens upload to logits)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * (PREFILLS + 1))]
        ev[0].record(stream)
        logits = model.forward(cache, prompt)
        ev[1].record(stream)
        for i in range(PREFILLS):
            cache.reset()
            ev[2 + 2 * i].record(stream)
            logits = model.forward(cache, prompt)
            ev[3 + 2 * i].record(stream)
        tok = int(torch.argmax(logits.float()).item())
        torch.cuda.synchronize()
        prefill_first_ms = ev[0].elapsed_time(ev[1])
        prefill_runs = sorted(ev[2 + 2 * i].elapsed_time(ev[3 + 2 * i]) for i in range(PREFILLS))
        prefill_ms = float(np.median(prefill_runs))
        log(f"prefill {args.prompt} tokens: first {prefill_first_ms:.1f} ms, warm median of {PREFILLS} "
            f"{prefill_ms:.2f} ms (runs {', '.join(f'{x:.2f}' for x in prefill_runs)})")
        # warmup (captures the decode graph), then rewind to the prompt
        t = tok
        for _ in range(args.warmup):
            t = model.decode_step(cache, t)
        cache.truncate(args.prompt)
        torch.cuda.synchronize()
        # timed region: exactly `steps` decode tokens from position 4096,
        # through the greedy decode loop (the prefill's token first, then one
        # graph replay per token, queued ahead of the token being checked)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = model.decode_greedy(cache, tok, args.steps + 1, eos=())
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        assert len(toks) == args.steps + 1 and cache.seq_len == args.prompt + args.steps
        # the same steps one synchronous bmx_qwen3_decode_step at a time: the
        # host reads each token before it launches the next step
        cache.truncate(args.prompt)
        t = tok
        sync_toks = [tok]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            t = model.decode_step(cache, t)
            sync_toks.append(t)
        torch.cuda.synchronize()
        dt_sync = time.perf_counter() - t0
        assert list(toks) == sync_toks, "queued and synchronous decode steps disagree"
    tok_s = args.steps / dt
    log(f"decode {args.steps} tokens at ctx {args.prompt}: {dt * 1000 / args.steps:.3f} ms/token, {tok_s:.1f} tok/s "
        f"(one synchronous step at a time: {dt_sync * 1000 / args.steps:.3f} ms/token)")
    model.close()
    del cache
    torch.cuda.empty_cache()

    # whole-step roofline: bytes each timed token reads (weights, and the
    # K / V of its context: token i of the timed region sits at position
    # prompt + i) over the measured time per token
    kv_per_pos = 2 * 2 * SHAPE_4B["layers"] * SHAPE_4B["n_kv_heads"] * SHAPE_4B["head_dim"]
    step_bytes = decode_weight_bytes(SHAPE_4B) + kv_per_pos * (args.prompt + (args.steps - 1) / 2.0)
    step_gbs = step_bytes * tok_s / 1e9
    step_roof = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                 "frac": round(step_gbs / HBM_PEAK_GBS, 4), "bytes_per_token": int(step_bytes),
                 "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1)}
    log(f"decode step: {step_bytes / 1e9:.3f} GB per token -> {step_gbs:.0f} GB/s "
        f"({100 * step_gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s; roofline {step_roof['roofline_tok_s']} tok/s)")

    att_us, att_bytes = time_decode_attention(bmx, torch)
    att_gbs = att_bytes / att_us / 1e3
    tr = traced_duration_us()
    roof = {"bound": "hbm", "achieved": round(att_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(att_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "kernel": f"decode attention (attn_decode_kernel: QK-norm, RoPE, KV write, split-key GQA, merge), "
                      f"Qwen3-4B heads, token at position {ATT_CTX}",
            "avg_launch_us": round(att_us, 3), "bytes_per_launch": att_bytes,
            "traffic_from": f"profiles/{TRAFFIC_PROFILE} (rocprofv3 --pmc; not measured in this run)",
            "trace_avg_us": tr, "trace_avg_us_from": f"profiles/{TRACE_PROFILE} (rocprofv3 kernel trace of "
                                                      f"bench.py --profile-roofline; not measured in this run)",
            "frac_trace": None if tr is None else round(att_bytes / tr / 1e3 / HBM_PEAK_GBS, 4)}
    log(f"decode attention at position {ATT_CTX}: {att_us:.2f} us per launch, {att_gbs:.0f} GB/s "
        f"({100 * att_gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)")

    sweep = []
    if not args.no_sweep:
        for (N, K) in QMV_SHAPES:
            us, nb = time_qmv(bmx, torch, N, K)
            gbs = nb / us / 1e3
            sweep.append({"N": N, "K": K, "us": round(us, 3), "GB/s": round(gbs, 1),
                          "frac": round(gbs / HBM_PEAK_GBS, 4), "launches": 1000})
            log(f"qmv N={N} K={K}: {us:.2f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)")

    qmm = [] if args.no_qmm_sweep else qmm_sweep(bmx, torch)
    spec = None if args.no_speculative else speculative_bench(bmx, torch)
    small = None if args.no_small else small_model_bench(bmx, torch, cpu=not args.no_cpu)
    moe = moe_bench(bmx, torch) if args.moe else []

    cpu = None
    if not args.no_cpu:
        host = host_info()
        v = cpu_baseline(args.cpu_tokens)
        cpu = {"value": round(v, 3), "unit": "tok/s", "cores": host["threads"], "kind": "port",
               "sample": f"{args.cpu_tokens} greedy decode tokens of the same Qwen3-4B shape at context 4096 "
                         f"(KV positions 0..4095 filled synthetically), oracle/ C restatement, OpenMP",
               "host": host}
        log(f"cpu baseline: {v:.3f} tok/s on {host['threads']} threads ({host})")

    out = {
        "metric": "decode tok/s Qwen3-4B-shape 4-bit bs1; qmv GB/s as % of HBM peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1000 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations, u4 weights (MLX affine gs64), fp32 accumulate",
        "data": "synthetic: seeded random-init weights N(0,0.02) quantized 4-bit, seeded random token ids",
        "config": {"workload": "Qwen3-4B-shape 4-bit greedy decode, batch 1, after a 4096-token prefill",
                   "prompt_tokens": args.prompt, "kv_cache": [36, 2, 8, max(cap, 4352), 128],
                   "prefill_ms": round(prefill_ms, 2), "prefill_first_call_ms": round(prefill_first_ms, 2),
                   "prefill_runs_ms": [round(x, 2) for x in prefill_runs],
                   "decode_step_sync_tok_s": round(args.steps / dt_sync, 2), "qmv_sweep": sweep, "qmm_sweep": qmm,
                   "speculative": spec, "qwen3_0_6b": small, "gather_qmm": moe},
        "roofline": roof,
        "step_roofline": step_roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
