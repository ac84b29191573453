"""Statistics of the paired A/B methodology (pure CPU: no GPU, no torch).

What a decision rests on (the policy of the reference's harness
paired-streaming-v2.3, cudalab/evaluator/stats.py:1-222; the thresholds,
record keys and reason key words are kept so that records and callers stay
comparable, the code is this build's own):

* Rounds, not samples.  Within a round the two variants are timed back to
  back on the same pool; a round contributes one speedup, parent /
  candidate (> 1: the candidate is faster).  Samples only feed the round's
  medians.
* Two guards, both symmetric (a sample or block that is too fast is as
  suspect as one that is too slow):
    - a timed sample outside [m / 1.5, m * 1.5], m the median of the last
      50 samples the guard accepted in the same block, is rejected;
    - a block whose filtered median lies outside [r / 1.15, r * 1.15], r
      the median of the same variant's earlier block medians, flags its
      round (once 3 earlier blocks exist).
  Both bounds are inclusive: a value exactly on a bound is accepted.  Every
  block keeps the raw and the filtered track, so a record can show what the
  guards changed (`filter_sensitive`).
* A fixed-seed percentile bootstrap of the median round speedup, so that a
  record's interval reproduces bit for bit: replicate b draws n indices with
  `random.Random(seed).randrange(n)` in sequence, and the bounds are the
  sorted replicates at int(alpha/2 * B) and int((1 - alpha/2) * B) - 1 (the
  reference's draw order and indices, so the same speedups give the same
  interval).

GPU clocks are not sampled inside a round on MI355X (amd-smi snapshots are
taken before and after a run, evaluator/gpu.py), so there is no clock
agreement check here.
"""
from __future__ import annotations

import math
import random
import statistics
from collections import Counter, deque
from typing import Iterable, Optional

BOOTSTRAP_SEED = 20260919
BOOTSTRAP_N = 10000
CI_ALPHA = 0.05

FILTER_LOG_DELTA = math.log(1.10)

SPIKE_FACTOR = 1.5
SPIKE_WINDOW = 50
CROSSBLOCK_FACTOR = 1.15
CROSSBLOCK_WARMUP = 3


def _side(value: float, center: float, factor: float) -> Optional[str]:
    """Which side of the band [center / factor, center * factor] `value`
    falls out of: "slow" above, "fast" below, None inside (bounds
    included)."""
    if value > center * factor:
        return "slow"
    if value < center / factor:
        return "fast"
    return None


# ------------------------------------------------------------ sample guard
class SampleGuard:
    """The sample-level guard of one block.  Samples are offered in timing
    order; each is judged against the median of the last `window` samples
    this guard accepted (the first sample is always accepted)."""

    def __init__(self, factor: float = SPIKE_FACTOR,
                 window: int = SPIKE_WINDOW) -> None:
        self.factor = factor
        self._recent: deque[float] = deque(maxlen=window)
        self.accepted: list[float] = []
        self.rejected: Counter[str] = Counter()

    def verdict(self, t_us: float) -> Optional[str]:
        """"fast" / "slow" if `t_us` would be rejected, else None (the
        guard's state is not changed)."""
        if not self._recent:
            return None
        return _side(t_us, statistics.median(self._recent), self.factor)

    def offer(self, t_us: float) -> Optional[str]:
        """Judge one sample and record it; returns the rejection side or
        None when accepted."""
        side = self.verdict(t_us)
        if side is None:
            self._recent.append(t_us)
            self.accepted.append(t_us)
        else:
            self.rejected[side] += 1
        return side


def apply_spike_guard(accepted: list[float], t_us: float,
                      spike_factor: float = SPIKE_FACTOR,
                      window: int = SPIKE_WINDOW) -> tuple[bool, Optional[str]]:
    """Stateless form of the sample guard: (accepted?, side) of `t_us`
    against the median of the last `window` entries of `accepted`."""
    side = (None if not accepted else
            _side(t_us, statistics.median(accepted[-window:]), spike_factor))
    return side is None, side


def block_stats(raw_samples_us: Iterable[float],
                spike_factor: float = SPIKE_FACTOR,
                window: int = SPIKE_WINDOW) -> dict:
    """Raw and filtered tracks of one block of timed samples."""
    raw = list(raw_samples_us)
    guard = SampleGuard(spike_factor, window)
    for t in raw:
        guard.offer(t)
    kept = guard.accepted
    n_out = guard.rejected["fast"] + guard.rejected["slow"]
    return {
        "median_us": statistics.median(kept) if kept else None,
        "raw_median_us": statistics.median(raw) if raw else None,
        "n_raw": len(raw),
        "n_accepted": len(kept),
        "n_rejected_fast": guard.rejected["fast"],
        "n_rejected_slow": guard.rejected["slow"],
        # the same counts under the field names of older records
        "n_clean": len(kept),
        "n_spike": n_out,
        "raw_samples_us": [round(t, 3) for t in raw],
        "accepted_samples_us": [round(t, 3) for t in kept],
    }


# ------------------------------------------------------------- block guard
def crossblock_flag(hist: list[float], med: Optional[float],
                    factor: float = CROSSBLOCK_FACTOR,
                    warmup: int = CROSSBLOCK_WARMUP) -> dict:
    """Judge a block's filtered median `med` against the median of the same
    variant's earlier block medians `hist` (a list the caller keeps per
    variant; `med` is appended after it is judged, so warm-up blocks enter
    the history too).  Nothing is judged before `warmup` earlier blocks
    exist, and a missing median is neither judged nor recorded."""
    out: dict = {"running_med_us": None, "ratio": None, "flagged": False,
                 "direction": None}
    if med is None:
        return out
    if len(hist) >= warmup:
        ref = statistics.median(hist)
        ratio = med / ref if ref > 0 else math.inf
        side = _side(ratio, 1.0, factor)
        out.update(running_med_us=round(ref, 3), ratio=round(ratio, 4),
                   flagged=side is not None, direction=side)
    hist.append(med)
    return out


def filter_sensitive(raw_speedup: Optional[float],
                     filtered_speedup: Optional[float],
                     log_delta: float = FILTER_LOG_DELTA) -> tuple[bool, str]:
    """Did the guards change the conclusion?  Yes when the raw and the
    filtered paired speedups lie strictly on opposite sides of 1.0, or their
    ratio is beyond exp(log_delta) either way.  A missing or non-positive
    speedup is not evaluated."""
    if not (raw_speedup and filtered_speedup
            and raw_speedup > 0 and filtered_speedup > 0):
        return False, ("not evaluated (未评估): raw or filtered speedup "
                       "missing or invalid")
    if (raw_speedup - 1.0) * (filtered_speedup - 1.0) < 0:
        return True, (f"direction flip (方向翻转): raw {raw_speedup:.4f} and "
                      f"filtered {filtered_speedup:.4f} lie on opposite "
                      "sides of 1.0")
    gap = abs(math.log(filtered_speedup) - math.log(raw_speedup))
    if gap > log_delta:
        return True, (f"|log(filtered/raw)| = {gap:.4f} > {log_delta:.4f} "
                      "(more than 10% apart)")
    return False, (f"within threshold (阈值内): |log difference| {gap:.4f} "
                   f"<= {log_delta:.4f}")


# --------------------------------------------------------- round statistics
def paired_speedups(parent_round_us: list[float],
                    candidate_round_us: list[float]) -> list[float]:
    """Per-round parent / candidate from the two variants' round medians."""
    if len(parent_round_us) != len(candidate_round_us):
        raise ValueError(f"paired lengths differ: {len(parent_round_us)} vs "
                         f"{len(candidate_round_us)}")
    bad = [(p, c) for p, c in zip(parent_round_us, candidate_round_us)
           if p <= 0 or c <= 0]
    if bad:
        p, c = bad[0]
        raise ValueError(f"non-positive time: parent={p} candidate={c}")
    return [p / c for p, c in zip(parent_round_us, candidate_round_us)]


_SUMMARY_KEYS = ("n", "median", "mean", "min", "max", "faster_count",
                 "faster_fraction")


def summarize(speedups: list[float]) -> dict:
    """Count, centre, spread and the share of rounds the candidate won."""
    if not speedups:
        return dict.fromkeys(_SUMMARY_KEYS) | {"n": 0, "faster_count": 0}
    wins = sum(s > 1.0 for s in speedups)
    r6 = lambda v: round(v, 6)  # noqa: E731
    return {"n": len(speedups), "median": r6(statistics.median(speedups)),
            "mean": r6(statistics.fmean(speedups)), "min": r6(min(speedups)),
            "max": r6(max(speedups)), "faster_count": wins,
            "faster_fraction": round(wins / len(speedups), 4)}


def bootstrap_ci(values: list[float], statistic: str = "median",
                 n_boot: int = BOOTSTRAP_N, alpha: float = CI_ALPHA,
                 seed: int = BOOTSTRAP_SEED) -> Optional[list[float]]:
    """Percentile bootstrap interval [lo, hi] of the median (or "mean") of
    `values`, or None for fewer than 3 values (draw order in the module
    docstring)."""
    n = len(values)
    if n < 3:
        return None
    stat = statistics.median if statistic == "median" else statistics.fmean
    draw = random.Random(seed).randrange
    reps = sorted(stat([values[draw(n)] for _ in range(n)])
                  for _ in range(n_boot))
    lo = reps[int((alpha / 2) * n_boot)]
    hi = reps[int((1.0 - alpha / 2) * n_boot) - 1]
    return [round(lo, 6), round(hi, 6)]
