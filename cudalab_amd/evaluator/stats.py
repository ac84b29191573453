"""Round-level paired statistics of the A/B methodology (pure CPU: no GPU,
no torch).

Restates `cudalab/evaluator/stats.py` (harness paired-streaming-v2.3):

* The unit of inference is the independent benchmark *round*, never the
  individual timed sample: within a round the two variants are measured
  back to back on the same tensors, and only round-level speedups
  (parent / candidate, > 1 means the candidate is faster) enter the
  statistics (:1-12, :170-199).
* Percentile bootstrap of the median round speedup with a fixed seed, so a
  record's CI is reproducible bit for bit (:202-222).  The resampling order
  (Python `random.Random(seed).randrange(n)`, n draws per replicate) and
  the percentile indices are kept exactly as the reference's, so the same
  speedups give the same interval.
* Symmetric guards (:26-143): a timed sample farther than a factor 1.5
  from the median of the last 50 accepted samples is rejected (fast and
  slow alike); a block whose filtered median is farther than 1.15 from the
  running median of that variant's earlier blocks invalidates the round
  (after 3 warm-up blocks).  Every block keeps raw and filtered statistics.
* Filter sensitivity (:146-167): raw and filtered speedups that fall on
  opposite sides of 1.0, or differ by more than 10% (|log ratio| >
  log 1.10), mark the record as filter-sensitive.
* The clock-agreement checks (:225-258) of the v0.2 harness, kept for old
  records (no timed round samples clocks any more).

Reason strings carry the reference's key words (方向翻转 / 阈值内 / 未评估)
next to the English text, because callers match them.
"""
from __future__ import annotations

import math
import random
import statistics

BOOTSTRAP_SEED = 20260919
BOOTSTRAP_N = 10000
CI_ALPHA = 0.05

FILTER_LOG_DELTA = math.log(1.10)

SPIKE_FACTOR = 1.5
SPIKE_WINDOW = 50
CROSSBLOCK_FACTOR = 1.15
CROSSBLOCK_WARMUP = 3


# ------------------------------------------------------------ sample guard
def apply_spike_guard(accepted: list[float], t_us: float,
                      spike_factor: float = SPIKE_FACTOR,
                      window: int = SPIKE_WINDOW) -> tuple[bool, str | None]:
    """Accept or reject one timed sample against the median of the last
    `window` accepted samples: (False, "slow") above ref * factor, (False,
    "fast") below ref / factor, else (True, None).  The thresholds are
    strict (a sample exactly at a threshold is accepted) and the first
    sample of a block is always accepted."""
    if not accepted:
        return True, None
    ref = statistics.median(accepted[-window:])
    if t_us > ref * spike_factor:
        return False, "slow"
    if t_us < ref / spike_factor:
        return False, "fast"
    return True, None


def block_stats(raw_samples_us: list[float],
                spike_factor: float = SPIKE_FACTOR,
                window: int = SPIKE_WINDOW) -> dict:
    """Raw and filtered statistics of one block of timed samples (the guard
    applied sample by sample, in order)."""
    kept: list[float] = []
    fast = slow = 0
    for t in raw_samples_us:
        ok, why = apply_spike_guard(kept, t, spike_factor, window)
        if ok:
            kept.append(t)
        elif why == "fast":
            fast += 1
        else:
            slow += 1
    return {
        "median_us": statistics.median(kept) if kept else None,
        "raw_median_us": (statistics.median(raw_samples_us)
                          if raw_samples_us else None),
        "n_raw": len(raw_samples_us),
        "n_accepted": len(kept),
        "n_rejected_fast": fast,
        "n_rejected_slow": slow,
        # field names older records used for the same counts
        "n_clean": len(kept),
        "n_spike": fast + slow,
        "raw_samples_us": [round(t, 3) for t in raw_samples_us],
        "accepted_samples_us": [round(t, 3) for t in kept],
    }


def crossblock_flag(hist: list[float], med: float | None,
                    factor: float = CROSSBLOCK_FACTOR,
                    warmup: int = CROSSBLOCK_WARMUP) -> dict:
    """Judge one block's filtered median `med` against the running median
    of the same variant's earlier blocks (`hist`, owned by the caller; med
    is appended after judging, warm-up blocks included).  Flags "slow"
    above median * factor and "fast" below median / factor once at least
    `warmup` blocks are in hist.  med None is neither judged nor
    appended."""
    info: dict = {"running_med_us": None, "ratio": None,
                  "flagged": False, "direction": None}
    if med is None:
        return info
    if len(hist) >= warmup:
        running = statistics.median(hist)
        ratio = med / running if running > 0 else float("inf")
        info["running_med_us"] = round(running, 3)
        info["ratio"] = round(ratio, 4)
        if ratio > factor:
            info["flagged"], info["direction"] = True, "slow"
        elif ratio < 1.0 / factor:
            info["flagged"], info["direction"] = True, "fast"
    hist.append(med)
    return info


def filter_sensitive(raw_speedup: float | None,
                     filtered_speedup: float | None,
                     log_delta: float = FILTER_LOG_DELTA) -> tuple[bool, str]:
    """Whether the guards changed the conclusion: the raw and filtered
    paired speedups lie strictly on opposite sides of 1.0, or
    |log(filtered / raw)| > log_delta.  Missing or non-positive inputs are
    not evaluated (False)."""
    if (raw_speedup is None or filtered_speedup is None
            or raw_speedup <= 0 or filtered_speedup <= 0):
        return False, "not evaluated (未评估): raw or filtered speedup missing or invalid"
    if (raw_speedup < 1.0 < filtered_speedup
            or filtered_speedup < 1.0 < raw_speedup):
        return True, (f"direction flip (方向翻转): raw {raw_speedup:.4f} and "
                      f"filtered {filtered_speedup:.4f} lie on opposite sides of 1.0")
    delta = abs(math.log(filtered_speedup / raw_speedup))
    if delta > log_delta:
        return True, (f"|log(filtered/raw)| = {delta:.4f} > {log_delta:.4f} "
                      f"(more than 10% apart)")
    return False, (f"within threshold (阈值内): |log difference| {delta:.4f} "
                   f"<= {log_delta:.4f}")


# --------------------------------------------------------- round statistics
def paired_speedups(parent_round_us: list[float],
                    candidate_round_us: list[float]) -> list[float]:
    """Per-round parent / candidate (> 1 = candidate faster).  The lists
    are the two variants' medians of the same rounds."""
    if len(parent_round_us) != len(candidate_round_us):
        raise ValueError(f"paired lengths differ: {len(parent_round_us)} vs "
                         f"{len(candidate_round_us)}")
    out = []
    for p, c in zip(parent_round_us, candidate_round_us):
        if p <= 0 or c <= 0:
            raise ValueError(f"non-positive time: parent={p} candidate={c}")
        out.append(p / c)
    return out


def summarize(speedups: list[float]) -> dict:
    if not speedups:
        return {"n": 0, "median": None, "mean": None, "min": None,
                "max": None, "faster_count": 0, "faster_fraction": None}
    faster = sum(1 for s in speedups if s > 1.0)
    return {
        "n": len(speedups),
        "median": round(statistics.median(speedups), 6),
        "mean": round(statistics.fmean(speedups), 6),
        "min": round(min(speedups), 6),
        "max": round(max(speedups), 6),
        "faster_count": faster,
        "faster_fraction": round(faster / len(speedups), 4),
    }


def bootstrap_ci(values: list[float], statistic: str = "median",
                 n_boot: int = BOOTSTRAP_N, alpha: float = CI_ALPHA,
                 seed: int = BOOTSTRAP_SEED) -> list[float] | None:
    """Percentile bootstrap CI [lo, hi] of the median (or mean) of
    `values`; None for fewer than 3 values."""
    n = len(values)
    if n < 3:
        return None
    rng = random.Random(seed)
    stat = statistics.median if statistic == "median" else statistics.fmean
    reps = []
    for _ in range(n_boot):
        reps.append(stat([values[rng.randrange(n)] for _ in range(n)]))
    reps.sort()
    lo = reps[int((alpha / 2) * n_boot)]
    hi = reps[int((1.0 - alpha / 2) * n_boot) - 1]
    return [round(lo, 6), round(hi, 6)]


# ------------------------------------------------ clock agreement (v0.2)
def check_dvfs_pair(clk_before, clk_after_first, clk_after_second,
                    parent_first: bool, tol: float) -> tuple:
    """A paired round's clock agreement: each variant's effective clock is
    the mean of the samples around its measurement; a relative difference
    above `tol` invalidates the round.  Returns (valid, reason,
    eff_parent, eff_candidate)."""
    if not (clk_before and clk_after_first and clk_after_second):
        return False, "no_clock_data", None, None
    first = (clk_before + clk_after_first) / 2.0
    second = (clk_after_first + clk_after_second) / 2.0
    eff_p, eff_c = (first, second) if parent_first else (second, first)
    mid = (eff_p + eff_c) / 2.0
    ok = abs(eff_p - eff_c) / mid <= tol if mid > 0 else False
    return ok, (None if ok else "INVALID_DVFS"), eff_p, eff_c


def check_dvfs_matrix(clks: list, tol: float) -> tuple:
    """A matrix round's clock agreement: the spread of the variants'
    effective clocks (means of adjacent samples) over their mean must not
    exceed `tol`.  Returns (valid, reason, effective_clocks)."""
    if not clks or not all(clks):
        return False, "no_clock_data", []
    effs = [(clks[i] + clks[i + 1]) / 2.0 for i in range(len(clks) - 1)]
    spread = (max(effs) - min(effs)) / statistics.fmean(effs)
    ok = spread <= tol
    return ok, (None if ok else "INVALID_DVFS"), effs
