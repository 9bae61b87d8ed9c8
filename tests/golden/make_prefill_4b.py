"""Writes tests/golden/qwen3_4b_prefill4096.npz: the oracle's last-row logits
after a 4096-token prefill of the whole Qwen3-4B-shaped model (36 layers,
hidden 2560, intermediate 9728, 32 q / 8 kv heads, vocabulary 151936;
random-init weights seed 42, sigma 0.02; prompt = fill_tokens(11, 4096)),
and what the oracle with every fp32 reduction reversed gives at the same
position (its L2 distance from the forward order and its argmax: the floor
that summation order alone sets).

The oracle needs about 16 minutes per pass on 8 cores for this, too long
for a test, so the result is kept as a fixture; the oracle is thread-count
deterministic (its reductions have a fixed order whatever the thread count),
so the fixture does not depend on the machine that wrote it.  Run from the
repository root after building the oracle (make -C oracle):

    python tests/golden/make_prefill_4b.py
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as orc  # noqa: E402

SHAPE = dict(hidden=2560, inter=9728, layers=36, n_heads=32, n_kv_heads=8, head_dim=128, vocab=151936)
MODEL_SEED, PROMPT_SEED, P = 42, 11, 4096
OUT = os.path.join(ROOT, "tests", "golden", "qwen3_4b_prefill4096.npz")


def main():
    om = orc.Qwen3(orc.make_config(**SHAPE), MODEL_SEED, 0.02)
    toks = orc.fill_tokens(PROMPT_SEED, P, SHAPE["vocab"])
    t0 = time.time()
    o = om.forward(om.new_cache(P), toks)
    print(f"forward order: {time.time() - t0:.0f} s", flush=True)
    t0 = time.time()
    with orc.reversed_accumulation():
        r = om.forward(om.new_cache(P), toks)
    print(f"reversed order: {time.time() - t0:.0f} s", flush=True)
    of = orc.bf16_to_f32(o).astype(np.float64)
    rf = orc.bf16_to_f32(r).astype(np.float64)
    floor = float(np.linalg.norm(rf - of) / np.linalg.norm(of))
    np.savez_compressed(OUT, logits=o, floor_l2=np.float64(floor), floor_argmax=np.int64(np.argmax(rf)),
                        rms_spread=np.float64(np.sqrt(np.mean((rf - of) ** 2))), model_seed=MODEL_SEED,
                        prompt_seed=PROMPT_SEED, prompt_len=P)
    print(f"wrote {OUT}: argmax {int(np.argmax(of))}, reversed argmax {int(np.argmax(rf))}, floor L2 {floor:.3e}")


if __name__ == "__main__":
    main()
