"""Experiment records and per-cell winner classification (pure CPU).

Restates `cudalab/evaluator/experiment.py`:

* One optimisation attempt is one JSON record, failed ones included;
  records get monotonic ids PREFIX-NNNN (:52-71).
* `classify_cell` (:74-200): winners are decided per (shape, dtype, cache
  mode) cell, never globally.  The winner is the variant with the lowest
  median over valid rounds; the runner-up / winner round-level paired
  ratios go through the fixed decision rules (correctness is gated
  elsewhere, so it counts as passed):
      KEEP      -> SIGNIFICANT_WINNER
      NEUTRAL   -> NO_UNIQUE_WINNER
      REJECT    -> NO_UNIQUE_WINNER
      UNSTABLE  -> UNSTABLE
  When the rounds carry raw (pre-guard) times, a different raw winner, or
  a raw top-2 ratio more than 10% from the filtered one, makes the cell
  filter-sensitive (UNSTABLE).  The raw side uses the same convention as
  the filtered side: the median of the per-round ratios.
"""
from __future__ import annotations

import json
import re
import statistics
from pathlib import Path

from . import decision as _decision
from . import stats as _stats

SIGNIFICANT_WINNER = "SIGNIFICANT_WINNER"
NO_UNIQUE_WINNER = "NO_UNIQUE_WINNER"
UNSTABLE = "UNSTABLE"

_STATUS = {
    _decision.KEEP: SIGNIFICANT_WINNER,
    _decision.NEUTRAL: NO_UNIQUE_WINNER,
    _decision.REJECT: NO_UNIQUE_WINNER,
    _decision.UNSTABLE: UNSTABLE,
}


def next_experiment_id(exp_dir: Path, prefix: str) -> str:
    """PREFIX-NNNN, one past the largest number already in exp_dir."""
    exp_dir = Path(exp_dir)
    exp_dir.mkdir(parents=True, exist_ok=True)
    pat = re.compile(rf"^{re.escape(prefix)}-(\d+)\.json$")
    nums = [int(m.group(1)) for p in exp_dir.glob(f"{prefix}-*.json")
            if (m := pat.match(p.name))]
    return f"{prefix}-{(max(nums) + 1 if nums else 1):04d}"


def save_experiment(record: dict, exp_dir: Path, prefix: str = "EXP") -> Path:
    exp_dir = Path(exp_dir)
    exp_dir.mkdir(parents=True, exist_ok=True)
    if not record.get("id"):
        record["id"] = next_experiment_id(exp_dir, prefix)
    path = exp_dir / f"{record['id']}.json"
    path.write_text(json.dumps(record, indent=2, ensure_ascii=False))
    return path


def _raw_track(variants, valid, winner, runner, filtered_median):
    """(raw medians, raw winner, filter_sensitive, reason) of a cell."""
    has_raw = all("us_raw" in r and r["us_raw"].get(winner) is not None
                  and r["us_raw"].get(runner) is not None for r in valid)
    if not has_raw:
        return None, None, False, "no raw data (records from before harness v2.3)"
    raw_medians = {}
    for v in variants:
        vals = [r["us_raw"][v] for r in valid
                if r.get("us_raw", {}).get(v) is not None]
        if vals:
            raw_medians[v] = round(statistics.median(vals), 3)
    ranked = sorted(raw_medians, key=raw_medians.get)
    winner_raw = ranked[0] if ranked else None
    if winner_raw is not None and winner_raw != winner:
        return (raw_medians, winner_raw, True,
                f"winner flip: raw winner {winner_raw!r} != filtered winner "
                f"{winner!r} (the guards changed the conclusion)")
    ratios = [r["us_raw"][runner] / r["us_raw"][winner] for r in valid]
    raw_ratio = statistics.median(ratios)
    fs, why = _stats.filter_sensitive(raw_ratio, filtered_median)
    return raw_medians, winner_raw, fs, why


def classify_cell(variants: list[str], rounds: list[dict],
                  min_valid_rounds: int = _decision.MIN_VALID_ROUNDS) -> dict:
    """Classify one matrix cell from its rounds ({valid, us: {variant: us},
    optional us_raw}).  Early exits (fewer than two comparable variants,
    too few valid rounds) carry no CI and no policy decision."""
    valid = [r for r in rounds if r["valid"]]
    medians = {}
    for v in variants:
        vals = [r["us"][v] for r in valid if v in r["us"]]
        if vals:
            medians[v] = round(statistics.median(vals), 3)
    ranked = sorted(medians, key=medians.get)
    out = {
        "valid_rounds": len(valid),
        "min_valid_rounds": min_valid_rounds,
        "all_variants_median_us": medians,
        "winner": ranked[0] if ranked else None,
        "runner_up": ranked[1] if len(ranked) > 1 else None,
        "median_ratio": None,
        "bootstrap_ci_95": None,
        "faster_rounds": None,
        "decision": None,
        "decision_rule": None,
        "statistical_relation": _decision.UNRESOLVED,
        "policy_decision": None,
        "status": None,
    }
    if len(ranked) < 2:
        out["status"] = (UNSTABLE if len(valid) < min_valid_rounds
                         else NO_UNIQUE_WINNER)
        out["decision_rule"] = "fewer than 2 comparable variants"
        return out
    winner, runner = ranked[0], ranked[1]
    if len(valid) < min_valid_rounds:
        out["status"] = UNSTABLE
        out["decision_rule"] = (f"valid rounds {len(valid)} < "
                                f"{min_valid_rounds} -> UNSTABLE")
        return out

    both = [r for r in valid if winner in r["us"] and runner in r["us"]]
    ratios = _stats.paired_speedups([r["us"][runner] for r in both],
                                    [r["us"][winner] for r in both])
    s = _stats.summarize(ratios)
    ci95 = _stats.bootstrap_ci(ratios)
    dec, detail = _decision.decide_v2(True, len(ratios), ratios, ci95)
    raw_medians, winner_raw, fs, why = _raw_track(variants, valid, winner,
                                                  runner, s["median"])
    out["all_variants_raw_median_us"] = raw_medians
    out["winner_raw"] = winner_raw
    dec, detail = _decision.apply_filter_gate(dec, detail, fs, why)
    out.update({
        "median_ratio": s["median"],
        "bootstrap_ci_95": ci95,
        "faster_rounds": f"{s['faster_count']}/{s['n']}",
        "decision": dec,
        "decision_rule": detail.get("rule"),
        "filter_sensitive": detail.get("filter_sensitive", False),
        "filter_sensitive_reason": detail.get("filter_sensitive_reason"),
        "statistical_relation": _decision.statistical_relation(ci95),
        "policy_decision": dec,
        "status": _STATUS[dec],
    })
    return out
