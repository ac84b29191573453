"""Fixed decision rules of the A/B methodology (pure CPU).

Restates `cudalab/evaluator/decision.py`.  A policy decision over the
round-level paired speedups (parent / candidate, > 1 = candidate faster),
the first matching rule winning (:13-21):

  1. correctness failed                  -> REJECT
  2. fewer than MIN_VALID_ROUNDS rounds  -> UNSTABLE
  3. median >= 1.05, >= 70% of rounds faster, CI95 lower bound > 1.00
                                         -> KEEP
  4. median <= 0.95, <= 30% of rounds faster, CI95 upper bound < 1.00
                                         -> REJECT
  5. otherwise                           -> NEUTRAL

then the filter gate (:23-31, :121-150): a filter-sensitive record (the
guards changed the conclusion) becomes UNSTABLE whatever rules 3-5 said,
with the original decision kept in the detail.  Separately,
`statistical_relation` states what the CI alone says (FASTER / SLOWER /
UNRESOLVED), independent of the 5% policy band (:33-44, :153-179).
"""
from __future__ import annotations

from . import stats as _stats

KEEP, REJECT, NEUTRAL, UNSTABLE = "KEEP", "REJECT", "NEUTRAL", "UNSTABLE"
FILTER_SENSITIVE = "FILTER_SENSITIVE"
FASTER, SLOWER, UNRESOLVED = "FASTER", "SLOWER", "UNRESOLVED"

MIN_VALID_ROUNDS = 5
KEEP_MEDIAN = 1.05
REJECT_MEDIAN = 0.95
KEEP_FASTER_FRAC = 0.70
REJECT_FASTER_FRAC = 0.30


def decide_v2(correctness_pass: bool, valid_rounds: int,
              speedups: list[float],
              ci95: list[float] | None) -> tuple[str, dict]:
    """(decision, detail); detail records the numbers behind the rule."""
    s = _stats.summarize(speedups)
    detail = {"correctness_pass": correctness_pass,
              "valid_rounds": valid_rounds,
              "min_valid_rounds": MIN_VALID_ROUNDS,
              "speedups": s, "ci95": ci95}

    def done(decision: str, rule: str):
        detail["rule"] = rule
        detail["decision"] = decision
        return decision, detail

    if not correctness_pass:
        return done(REJECT, "correctness FAIL -> REJECT (unconditional)")
    if valid_rounds < MIN_VALID_ROUNDS:
        return done(UNSTABLE, f"valid rounds {valid_rounds} < {MIN_VALID_ROUNDS} "
                              "-> UNSTABLE (unstable environment, no KEEP/REJECT)")
    if s["median"] is None:
        return done(UNSTABLE, "no valid speedup samples -> UNSTABLE")
    frac = s["faster_fraction"]
    lo = ci95[0] if ci95 else None
    hi = ci95[1] if ci95 else None
    if (s["median"] >= KEEP_MEDIAN and frac is not None
            and frac >= KEEP_FASTER_FRAC and lo is not None and lo > 1.00):
        return done(KEEP, f"median {s['median']:.4f} >= {KEEP_MEDIAN} AND "
                          f"{s['faster_count']}/{s['n']} rounds faster "
                          f"(>= {KEEP_FASTER_FRAC:.0%}) AND CI95 lower "
                          f"{lo:.4f} > 1.00 -> KEEP")
    if (s["median"] <= REJECT_MEDIAN and frac is not None
            and frac <= REJECT_FASTER_FRAC and hi is not None and hi < 1.00):
        return done(REJECT, f"median {s['median']:.4f} <= {REJECT_MEDIAN} AND "
                            f"{s['faster_count']}/{s['n']} rounds faster "
                            f"(<= {REJECT_FASTER_FRAC:.0%}) AND CI95 upper "
                            f"{hi:.4f} < 1.00 -> REJECT")
    return done(NEUTRAL, f"median {s['median']:.4f} within ({REJECT_MEDIAN}, "
                         f"{KEEP_MEDIAN}) or mixed rounds ({s['faster_count']}/"
                         f"{s['n']} faster) or CI95 {ci95} not excluding 1.00 "
                         "-> NEUTRAL")


def apply_filter_gate(decision: str, detail: dict, filter_sensitive: bool,
                      reason: str) -> tuple[str, dict]:
    """KEEP, REJECT and NEUTRAL become UNSTABLE when the record is
    filter-sensitive; UNSTABLE stays.  Returns a new detail dict (the input
    is not modified) with filter_sensitive / filter_sensitive_reason and,
    on a downgrade, original_decision and the new rule."""
    out = dict(detail)
    out["filter_sensitive"] = bool(filter_sensitive)
    out["filter_sensitive_reason"] = reason
    if filter_sensitive and decision in (KEEP, REJECT, NEUTRAL):
        out["original_decision"] = decision
        out["rule"] = (f"FILTER_SENSITIVE: {reason} -- {decision} downgraded to "
                       "UNSTABLE (the guards changed the conclusion; no "
                       "KEEP/REJECT/NEUTRAL)")
        return UNSTABLE, out
    return decision, out


def statistical_relation(ci95: list[float] | None) -> str:
    """FASTER if the CI95 lower bound > 1.00, SLOWER if the upper bound
    < 1.00, else (CI touching or containing 1.00, or missing) UNRESOLVED."""
    if ci95:
        lo, hi = float(ci95[0]), float(ci95[1])
        if lo > 1.00:
            return FASTER
        if hi < 1.00:
            return SLOWER
    return UNRESOLVED
