"""Frame-by-frame comparison of GPU greedy frames with the oracle run
teacher-forced by the GPU's own codes (shared by the GPU model and engine
tests).

For each frame of a voice the oracle runs the same local head fed the GPU's
codes (or_local_logits) with the GPU's repetition history, so every code of
every frame is compared, also after a near tie:
- with the GPU's own logits at hand, the GPU's code must be exactly the
  penalised argmax of those logits (penalty applied as the double 1.2) and
  the logits must be within the bar of the oracle's;
- the GPU's code must equal the oracle's penalised argmax, or else the
  oracle's margin between its choice and the GPU's must be at most 2.4 times
  the largest logit difference on that channel (the most a difference that
  small can move a penalised comparison), or the given bar without logits;
- the continue flag follows the same rule on the text decision.
Near ties are counted and printed.
"""
import numpy as np

from oracle import oracle
from conftest import say

PENALTY = 1.2


def _penalised(v):
    v = float(v)
    return v * PENALTY if v < 0 else v / PENALTY


class FrameCheck:
    """Per-voice repetition history and running counts for the comparison
    of GPU frames with the teacher-forced oracle."""

    def __init__(self, n_voices):
        self.seen = [[set() for _ in range(16)] for _ in range(n_voices)]
        self.codes_equal = self.codes_tied = self.flags_equal = self.flags_tied = 0
        self.max_logit_diff = self.max_text_diff = 0.0

    def frame(self, v, label, codes, cont, or_text2, or_logits, tol, gpu_text2=None,
              gpu_logits=None, bar=None):
        """Voice v's frame: the GPU chose `codes` / `cont`; the oracle ran the
        same frame teacher-forced with `codes`.  With the GPU's own logits the
        GPU's choices are first checked against them exactly."""
        if gpu_text2 is not None:
            d = float(np.abs(gpu_text2 - or_text2).max())
            self.max_text_diff = max(self.max_text_diff, d)
            assert d < tol, f"{label}: text decision differs by {d}"
            assert bool(cont) == (gpu_text2[1] >= gpu_text2[0]), f"{label}: flag vs own dot products"
            bar_t = 2 * d
        else:
            bar_t = bar
        or_cont = or_text2[1] >= or_text2[0]
        if bool(cont) == or_cont:
            self.flags_equal += 1
        else:
            gap = abs(or_text2[1] - or_text2[0])
            assert gap <= bar_t, f"{label}: continue flag differs, oracle gap {gap:.3e}"
            self.flags_tied += 1
            say(f"  {label}: near tie on the continue decision ({gap:.2e})")
        if not cont:
            return
        seen = self.seen[v]
        for ch in range(16):
            mask = sorted(seen[ch])
            g = int(codes[ch])
            if gpu_logits is not None:
                d = float(np.abs(gpu_logits[ch] - or_logits[ch]).max())
                self.max_logit_diff = max(self.max_logit_diff, d)
                assert d < tol, f"{label} ch {ch}: logits differ by {d}"
                own = oracle.argmax_penalty(gpu_logits[ch], mask, PENALTY)[0]
                assert own == g, f"{label} ch {ch}: GPU chose {g}, its own logits give {own}"
                bar_c = 2.4 * d
            else:
                bar_c = bar
            tok, best, _ = oracle.argmax_penalty(or_logits[ch], mask, PENALTY)
            if tok == g:
                self.codes_equal += 1
            else:
                s = or_logits[ch][g]
                s = _penalised(s) if g in seen[ch] else float(s)
                margin = best - s
                assert margin <= bar_c, (
                    f"{label} ch {ch}: GPU code {g}, oracle {tok}, oracle margin {margin:.3e} > {bar_c:.3e}")
                self.codes_tied += 1
                say(f"  {label} ch {ch}: near tie, GPU {g} vs oracle {tok} (margin {margin:.2e})")
            seen[ch].add(g)

    def summary(self, label):
        say(f"  {label}: {self.codes_equal} codes equal to the oracle's choice, {self.codes_tied} near "
            f"ties; flags {self.flags_equal} equal, {self.flags_tied} near ties; max |logits diff| "
            f"{self.max_logit_diff:.2e}, max |text diff| {self.max_text_diff:.2e}")
