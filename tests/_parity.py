"""End-to-end logits parity statistics shared by the model tests.

Per position: the L2 relative error of the GPU logits against the oracle's,
and the same for the oracle run with its accumulation order reversed (the
spread fp32 summation order alone causes through the layers: the floor no
implementation can be held below), plus greedy top-1 agreement.  The bar:
every position within max(E2E_TOL, FLOOR_FACTOR x the largest floor);
exact agreement on every position whose oracle top-2 margin is far above
the measured spread and above the bf16 resolution of the top logit
(decided positions, not near-ties: two logits a couple of bf16 steps apart
can round to one value, where the argmax's first-index rule decides); and,
over at least
MIN_POSITIONS positions, top-1 agreement of at least min(E2E_TOP1, the
reordered oracle's own agreement), less two standard deviations of the
oracle's own flip count (flips are coin tosses at near-ties).  The
reordered oracle reverses every fp32 reduction it has (GEMV, GEMM, SDPA,
RMSNorm).
"""
import numpy as np

from _util import bf16_to_f32, l2_rel_err

E2E_TOL = 2e-2       # north-star logits bar (L2 relative)
E2E_TOP1 = 0.99      # north-star greedy top-1 agreement
FLOOR_FACTOR = 1.5   # GPU spread allowed over the oracle's own reordering spread
MIN_POSITIONS = 64   # positions for the aggregate top-1 bar
BF16_STEPS = 3       # a decided position's oracle top-2 gap exceeds this many bf16 steps of its top logit
                     # (a GPU/oracle disagreement at a gap of 2-3 steps was seen at context 20000)


def _f32(bits):
    return bf16_to_f32(bits).astype(np.float64)


class Parity:
    """Per-position logits statistics: GPU vs oracle and reordered oracle vs
    oracle."""

    def __init__(self, name):
        self.name = name
        self.err, self.floor, self.agree, self.agree_floor, self.margin, self.resolved = [], [], [], [], [], []

    def add(self, g_bits, o_bits, r_bits):
        g = _f32(g_bits).reshape(-1, o_bits.shape[-1])
        o = _f32(o_bits).reshape(-1, o_bits.shape[-1])
        r = _f32(r_bits).reshape(-1, o_bits.shape[-1])
        for gi, oi, ri in zip(g, o, r):
            self.err.append(l2_rel_err(gi, oi))
            self.floor.append(l2_rel_err(ri, oi))
            self.agree.append(int(np.argmax(gi) == np.argmax(oi)))
            self.agree_floor.append(int(np.argmax(ri) == np.argmax(oi)))
            top2 = np.partition(oi, -2)[-2:]
            self.margin.append(float((top2[1] - top2[0]) / (np.linalg.norm(oi) / np.sqrt(oi.size))))
            # bf16 spacing at the top logit: 2^(exponent - 7)
            ulp = 2.0 ** (np.floor(np.log2(max(abs(top2[1]), 1e-30))) - 7)
            self.resolved.append(bool(top2[1] - top2[0] > BF16_STEPS * ulp))

    def check(self):
        err, floor = np.array(self.err), np.array(self.floor)
        agree, agree_f = np.array(self.agree), np.array(self.agree_floor)
        margin = np.array(self.margin)
        # positions whose top-2 margin (in units of the logits' rms) is well
        # above the spread the reordering causes are decided, not near-ties
        decided = (margin > 4.0 * max(float(np.max(floor)), float(np.max(err)))) & np.array(self.resolved, bool)
        bar = max(E2E_TOL, FLOOR_FACTOR * float(np.max(floor)))
        print(f"[{self.name}] {len(err)} positions: GPU-vs-oracle L2 max {err.max():.3e} mean {err.mean():.3e}; "
              f"reordered-oracle floor max {floor.max():.3e} mean {floor.mean():.3e}; bar {bar:.3e}; "
              f"top-1 GPU {agree.mean():.3f} floor {agree_f.mean():.3f}; decided positions {decided.sum()} "
              f"(top-1 there GPU {agree[decided].mean() if decided.any() else 1:.3f})", flush=True)
        assert err.max() <= bar, (err.max(), bar)
        # every decided position agrees; the aggregate agreement is held to
        # the bar once there are enough positions for it to mean something.
        # Flips happen only at near-ties, each one a coin toss, so the floor's
        # own flip count is a counting estimate: the slack is two standard
        # deviations of it (at least one position).
        if decided.any():
            assert agree[decided].all()
        n = len(err)
        if n >= MIN_POSITIONS:
            flips_floor = n - int(agree_f.sum())
            slack = max(1.0, 2.0 * np.sqrt(max(1, flips_floor))) / n
            assert agree.mean() >= min(E2E_TOP1, agree_f.mean()) - slack - 1e-9, (agree.mean(), agree_f.mean(), slack)
        return err, floor
