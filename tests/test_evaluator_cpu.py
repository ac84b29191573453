"""CPU tests of the A/B methodology (cudalab_amd.evaluator.stats / decision /
experiment, and the round logic of bench_pair / bench_matrix with synthetic
blocks).  The cases restate the reference's own evaluator tests
(tests/test_evaluator_cpu.py and tests/test_evaluator_v23_cpu.py): the
same inputs must give the same verdicts."""
from __future__ import annotations

import math
import random
import statistics

import pytest

from cudalab_amd.evaluator import decision as D
from cudalab_amd.evaluator import experiment as E
from cudalab_amd.evaluator import stats as S


# ----------------------------------------------------------- constants
def test_fixed_constants():
    assert (S.SPIKE_FACTOR, S.SPIKE_WINDOW) == (1.5, 50)
    assert (S.CROSSBLOCK_FACTOR, S.CROSSBLOCK_WARMUP) == (1.15, 3)
    assert abs(S.FILTER_LOG_DELTA - math.log(1.10)) < 1e-15
    assert (S.BOOTSTRAP_SEED, S.BOOTSTRAP_N, S.CI_ALPHA) == (20260919, 10000, 0.05)
    assert (D.MIN_VALID_ROUNDS, D.KEEP_MEDIAN, D.REJECT_MEDIAN) == (5, 1.05, 0.95)
    assert (D.KEEP_FASTER_FRAC, D.REJECT_FASTER_FRAC) == (0.70, 0.30)


# ------------------------------------------------ paired statistics (v0.2)
def test_paired_speedups():
    assert S.paired_speedups([2.0, 4.0], [1.0, 2.0]) == [2.0, 2.0]
    with pytest.raises(ValueError):
        S.paired_speedups([1.0], [1.0, 2.0])
    with pytest.raises(ValueError):
        S.paired_speedups([1.0, 0.0], [1.0, 1.0])


def test_summarize():
    s = S.summarize([1.10, 1.11, 1.09, 1.12, 1.10])
    assert s["n"] == 5 and abs(s["median"] - 1.10) < 1e-9
    assert s["faster_count"] == 5 and s["faster_fraction"] == 1.0
    assert (s["min"], s["max"]) == (1.09, 1.12)
    e = S.summarize([])
    assert e["n"] == 0 and e["median"] is None


def test_bootstrap_deterministic_and_sane():
    vals = [1.10, 1.09, 1.11, 1.10, 1.08, 1.12, 1.095]
    ci = S.bootstrap_ci(vals)
    assert ci == S.bootstrap_ci(vals)
    S.bootstrap_ci(vals, seed=12345)            # another seed must not fail
    lo, hi = ci
    assert lo <= 1.10 <= hi and lo > 1.00
    assert S.bootstrap_ci([1.1, 0.9]) is None   # fewer than 3 values


def test_bootstrap_matches_an_independent_restatement():
    """The CI equals a from-scratch percentile bootstrap with the same
    generator, draw order and percentile indices (so records computed here
    and by the reference agree on the same speedups)."""
    import random
    vals = [1.03, 0.97, 1.21, 1.08, 1.11, 0.99, 1.05, 1.02, 1.30]
    rng = random.Random(20260919)
    reps = sorted(statistics.median([vals[rng.randrange(len(vals))]
                                     for _ in range(len(vals))])
                  for _ in range(10000))
    assert S.bootstrap_ci(vals) == [round(reps[250], 6), round(reps[9749], 6)]
    rng = random.Random(7)
    reps = sorted(statistics.fmean([vals[rng.randrange(len(vals))]
                                    for _ in range(len(vals))])
                  for _ in range(10000))
    assert S.bootstrap_ci(vals, statistic="mean", seed=7) == \
        [round(reps[250], 6), round(reps[9749], 6)]


def test_sample_guard_matches_the_stateless_guard():
    """The block tracker and the one-sample function judge alike: random
    sample streams with spikes both ways, fed sample by sample."""
    rng = random.Random(3)
    for trial in range(200):
        kept, sides = [], []
        guard = S.SampleGuard()
        for i in range(rng.randint(1, 160)):
            t = rng.uniform(9.0, 11.0) * rng.choice([1, 1, 1, 1.6, 1 / 1.6, 1.49])
            ok, side = S.apply_spike_guard(kept, t)
            assert guard.verdict(t) == side
            assert guard.offer(t) == side
            if ok:
                kept.append(t)
            else:
                sides.append(side)
        assert guard.accepted == kept
        assert guard.rejected["fast"] == sides.count("fast")
        assert guard.rejected["slow"] == sides.count("slow")


def test_clock_agreement_helpers_are_gone():
    """MI355X rounds sample no clocks: no clock-agreement helper remains."""
    assert not hasattr(S, "check_dvfs_pair") and not hasattr(S, "check_dvfs_matrix")


# ---------------------------------------------------- decision rules (v0.2)
@pytest.mark.parametrize("speedups,want", [
    ([1.10, 1.11, 1.09, 1.12, 1.10], D.KEEP),
    ([1.01, 0.99, 1.02, 0.98, 1.00], D.NEUTRAL),
    ([0.90, 0.91, 0.89, 0.92, 0.90], D.REJECT),
    ([1.30, 0.80, 1.28, 0.82, 1.31], D.NEUTRAL),      # CI contains 1.00
    ([1.02, 1.03, 1.01, 1.04, 1.02], D.NEUTRAL),      # +2%: inside the band
    ([0.94, 0.95, 0.93, 0.96, 1.01], D.NEUTRAL),      # REJECT needs CI < 1.00
])
def test_decide_v2(speedups, want):
    dec, detail = D.decide_v2(True, len(speedups), speedups, S.bootstrap_ci(speedups))
    assert dec == want, detail


def test_decide_v2_gates():
    assert D.decide_v2(True, 2, [1.5, 1.6], None)[0] == D.UNSTABLE
    strong = [1.20, 1.21, 1.19, 1.22, 1.20]
    assert D.decide_v2(False, 5, strong, S.bootstrap_ci(strong))[0] == D.REJECT
    dec, detail = D.decide_v2(True, 9, [1.1] * 9, None)      # no CI: no KEEP
    assert dec == D.NEUTRAL and "rule" in detail


# ------------------------------------------------------- symmetric guards
def test_spike_guard_symmetric_and_strict():
    base = [10.0] * 50
    assert S.apply_spike_guard(base, 15.1) == (False, "slow")
    assert S.apply_spike_guard(base, 14.9) == (True, None)
    assert S.apply_spike_guard(base, 15.0) == (True, None)
    assert S.apply_spike_guard(base, 6.5) == (False, "fast")
    assert S.apply_spike_guard(base, 6.7) == (True, None)
    assert S.apply_spike_guard(base, 10.0 / 1.5) == (True, None)
    assert S.apply_spike_guard([], 1e9) == (True, None)
    assert S.apply_spike_guard([], 1e-9) == (True, None)


def test_spike_guard_window_is_last_50_accepted():
    hist = [10.0] * 60 + [11.0] * 40
    assert S.apply_spike_guard(hist, 16.5) == (True, None)
    assert S.apply_spike_guard(hist, 16.6) == (False, "slow")


def test_crossblock_guard():
    h = [10.0] * 3
    info = S.crossblock_flag(h, 11.6)
    assert info["flagged"] and info["direction"] == "slow"
    assert abs(info["ratio"] - 1.16) < 1e-9 and h[-1] == 11.6
    info = S.crossblock_flag([10.0] * 3, 8.6)
    assert info["flagged"] and info["direction"] == "fast"
    for med in (11.4, 8.7):
        info = S.crossblock_flag([10.0] * 3, med)
        assert not info["flagged"] and info["direction"] is None
    up = S.crossblock_flag([10.0] * 3, 10.0 * 1.16)
    dn = S.crossblock_flag([10.0] * 3, 10.0 / 1.16)
    assert (up["direction"], dn["direction"]) == ("slow", "fast")
    h = []
    for _ in range(3):
        info = S.crossblock_flag(h, 11.6)
        assert not info["flagged"] and info["ratio"] is None
    assert not S.crossblock_flag(h, 11.6)["flagged"] and len(h) == 4
    h = [10.0] * 3
    info = S.crossblock_flag(h, None)
    assert not info["flagged"] and info["ratio"] is None and len(h) == 3


def test_block_stats_tracks():
    st = S.block_stats([10.0] * 50 + [6.5] * 50)
    assert (st["n_raw"], st["n_accepted"]) == (100, 50)
    assert (st["n_rejected_fast"], st["n_rejected_slow"]) == (50, 0)
    assert st["raw_median_us"] == 8.25 and st["median_us"] == 10.0
    assert (st["n_clean"], st["n_spike"]) == (50, 50)
    st = S.block_stats([10.0] * 50 + [15.1] * 50)
    assert (st["n_rejected_fast"], st["n_rejected_slow"]) == (0, 50)
    assert st["raw_median_us"] == 12.55 and st["median_us"] == 10.0
    st = S.block_stats([])
    assert st["median_us"] is None and st["raw_median_us"] is None
    st = S.block_stats([10.0] * 100)
    assert st["n_accepted"] == 100 and st["raw_median_us"] == st["median_us"] == 10.0
    assert st["raw_samples_us"] == st["accepted_samples_us"] == [10.0] * 100


def test_guards_have_no_variant_bias():
    fast = [10.0] * 50 + [6.5] * 50
    slow = [10.0] * 50 + [15.1] * 50
    pa, ca = S.block_stats(fast), S.block_stats(slow)
    pb, cb = S.block_stats(slow), S.block_stats(fast)
    assert pa["median_us"] / ca["median_us"] == 1.0 == pb["median_us"] / cb["median_us"]
    ra = pa["raw_median_us"] / ca["raw_median_us"]
    rb = pb["raw_median_us"] / cb["raw_median_us"]
    assert abs(ra * rb - 1.0) < 1e-9 and ra < 1.0 < rb


# --------------------------------------------------- filter sensitivity
def test_filter_sensitive():
    ok, why = S.filter_sensitive(0.6846, 1.1111)
    assert ok and "翻转" in why
    assert S.filter_sensitive(1.20, 0.90)[0]
    ok, why = S.filter_sensitive(1.10, 1.11)
    assert not ok and "阈值内" in why
    ok, why = S.filter_sensitive(1.00, 1.11)
    assert ok and "log" in why
    assert not S.filter_sensitive(1.00, 1.10)[0]           # exactly log(1.10)
    ok, why = S.filter_sensitive(None, 1.11)
    assert not ok and "未评估" in why
    assert not S.filter_sensitive(0.0, 1.11)[0]


def test_filter_gate():
    dec, detail = D.decide_v2(True, 9, [1.1111] * 9, [1.1111, 1.1111])
    assert dec == D.KEEP
    before = dict(detail)
    dec2, d2 = D.apply_filter_gate(dec, detail, True, "方向翻转: constructed")
    assert dec2 == D.UNSTABLE and d2["original_decision"] == D.KEEP
    assert d2["filter_sensitive"] and "FILTER_SENSITIVE" in d2["rule"]
    assert detail == before                               # input untouched
    dec, detail = D.decide_v2(True, 9, [0.80] * 9, [0.80, 0.80])
    assert dec == D.REJECT
    assert D.apply_filter_gate(dec, detail, True, "winner flip")[0] == D.UNSTABLE
    dec, detail = D.decide_v2(True, 9, [1.02] * 9, [1.0, 1.04])
    assert dec == D.NEUTRAL
    dec2, d2 = D.apply_filter_gate(dec, detail, False, "阈值内")
    assert dec2 == D.NEUTRAL and "original_decision" not in d2
    for raw in (1.15, 0.85):                   # NEUTRAL + sensitive -> UNSTABLE
        sens, why = S.filter_sensitive(raw, 1.02)
        assert sens
        dec2, d2 = D.apply_filter_gate(dec, detail, sens, why)
        assert dec2 == D.UNSTABLE and d2["original_decision"] == D.NEUTRAL
    dec, detail = D.decide_v2(True, 9, [1.1111] * 9, [1.1111, 1.1111])
    dec2, d2 = D.apply_filter_gate(dec, detail, False, "阈值内")
    assert dec2 == D.KEEP and not d2["filter_sensitive"]


def test_constructed_filter_sensitive_end_to_end():
    p = S.block_stats([10.0] * 50 + [6.5] * 50)
    c = S.block_stats([9.0] * 50 + [15.1] * 50)
    assert (p["raw_median_us"], p["median_us"]) == (8.25, 10.0)
    assert (c["raw_median_us"], c["median_us"]) == (12.05, 9.0)
    raw = S.summarize([p["raw_median_us"] / c["raw_median_us"]] * 9)["median"]
    flt_sp = [p["median_us"] / c["median_us"]] * 9
    flt = S.summarize(flt_sp)["median"]
    assert raw < 1.0 < flt
    sens, why = S.filter_sensitive(raw, flt)
    assert sens
    dec, detail = D.decide_v2(True, 9, flt_sp, S.bootstrap_ci(flt_sp))
    assert dec == D.KEEP
    dec2, d2 = D.apply_filter_gate(dec, detail, sens, why)
    assert dec2 == D.UNSTABLE and d2["original_decision"] == D.KEEP


# ---------------------------------------------- statistical relation
def test_statistical_relation():
    assert D.statistical_relation([1.01, 1.20]) == D.FASTER
    assert D.statistical_relation([1.001, 1.04]) == D.FASTER
    assert D.statistical_relation([0.80, 0.99]) == D.SLOWER
    assert D.statistical_relation([0.95, 0.999]) == D.SLOWER
    for ci in ([0.98, 1.02], [1.00, 1.20], [0.80, 1.00], None):
        assert D.statistical_relation(ci) == D.UNRESOLVED
    assert D.decide_v2(True, 9, [1.01] * 9, [1.001, 1.04])[0] == D.NEUTRAL


# ----------------------------------------------------- classify_cell
def _bimodal_rounds():
    raws = [(10.0, 10.6), (10.0, 10.6), (10.0, 10.6), (10.0, 11.7),
            (50.0, 50.0), (50.0, 50.0), (50.0, 50.0)]
    return raws, [{"valid": True, "us": {"w": 10.0, "r": 10.6},
                   "us_raw": {"w": w, "r": r}} for w, r in raws]


def test_classify_cell_raw_convention_is_median_of_round_ratios():
    raws, rounds = _bimodal_rounds()
    across = (statistics.median(r for _, r in raws)
              / statistics.median(w for w, _ in raws))
    assert abs(across - 1.17) < 1e-9 and S.filter_sensitive(across, 1.06)[0]
    out = E.classify_cell(["w", "r"], rounds)
    assert not out["filter_sensitive"]
    assert out["decision"] == D.KEEP and out["status"] == E.SIGNIFICANT_WINNER
    assert (out["winner"], out["runner_up"], out["winner_raw"]) == ("w", "r", "w")
    assert out["all_variants_raw_median_us"] == {"w": 10.0, "r": 11.7}
    assert out["statistical_relation"] == D.FASTER and out["policy_decision"] == D.KEEP


def test_classify_cell_relation_policy_and_early_exits():
    out = E.classify_cell(["w", "r"], [{"valid": True, "us": {"w": 10.0, "r": 10.1}}
                                       for _ in range(9)])
    assert out["statistical_relation"] == D.FASTER
    assert out["policy_decision"] == D.NEUTRAL and out["status"] == E.NO_UNIQUE_WINNER
    out = E.classify_cell(["w"], [{"valid": True, "us": {"w": 10.0}}] * 9)
    assert out["statistical_relation"] == D.UNRESOLVED and out["policy_decision"] is None
    assert out["status"] == E.NO_UNIQUE_WINNER
    out = E.classify_cell(["w", "r"], [{"valid": False, "us": {}}] * 3)
    assert out["statistical_relation"] == D.UNRESOLVED and out["policy_decision"] is None
    assert out["status"] == E.UNSTABLE


def test_classify_cell_winner_flip_is_unstable():
    rounds = [{"valid": True, "us": {"a": 10.0, "b": 11.0},
               "us_raw": {"a": 12.0, "b": 11.0}} for _ in range(9)]
    out = E.classify_cell(["a", "b"], rounds)
    assert out["winner"] == "a" and out["winner_raw"] == "b"
    assert out["filter_sensitive"] and out["policy_decision"] == D.UNSTABLE
    assert out["status"] == E.UNSTABLE and "winner flip" in out["filter_sensitive_reason"]


def test_analyze_shape_winners_delegates():
    from cudalab_amd.evaluator.bench import analyze_shape_winners
    rec = {"shape": [128, 256], "dtype": "float16", "cache_mode": "streaming",
           "variants": ["a", "b"],
           "rounds": [{"valid": True, "us": {"a": 10.0, "b": 10.08},
                       "us_raw": {"a": 10.0, "b": 10.08}} for _ in range(9)]}
    [w] = analyze_shape_winners([rec])
    want = E.classify_cell(rec["variants"], rec["rounds"])
    for k in want:
        assert w[k] == want[k], k
    assert (w["shape"], w["dtype"], w["cache_mode"]) == ([128, 256], "float16", "streaming")
    assert w["statistical_relation"] == D.FASTER and w["policy_decision"] == D.NEUTRAL


def test_experiment_ids_and_save(tmp_path):
    assert E.next_experiment_id(tmp_path, "INT4GEMV") == "INT4GEMV-0001"
    p = E.save_experiment({"what": 1}, tmp_path, "INT4GEMV")
    assert p.name == "INT4GEMV-0001.json"
    (tmp_path / "INT4GEMV-0007.json").write_text("{}")
    (tmp_path / "INT4GEMV-x.json").write_text("{}")
    assert E.next_experiment_id(tmp_path, "INT4GEMV") == "INT4GEMV-0008"
    rec = {"id": "KEEP-ME"}
    assert E.save_experiment(rec, tmp_path).name == "KEEP-ME.json"


# ------------------------------- engine round logic with synthetic blocks
class _FakeOp:
    name = "fake"

    def variants(self, ext):
        return ["a", "b", "c"]

    def unsafe_variants(self, ext):
        return ["q"]

    def make_bench_pool(self, M, K, dtype, mode, seed, pool_size):
        from cudalab_amd.evaluator.bench import BenchPool
        return BenchPool(xs=[0], outs=[0], pool_size=1, working_set_bytes=1,
                         element_size=2, mode="hot", launch=lambda *a: None)

    def algorithmic_bytes(self, M, K, es):
        return 1_000_000


class _FakeExt:
    def aliases(self):
        return {"alias_of_a": "a"}


def _patch_engine(monkeypatch, times):
    """measure_block returns blocks of 60 identical samples with the
    per-variant time taken from `times` (a dict of iterators)."""
    from cudalab_amd.evaluator import bench as B
    calls = []

    def fake_block(pool, ext, v, warmup, iters, batch, caliber="native"):
        calls.append(v)
        t = next(times[v])
        return S.block_stats([t] * 60)
    monkeypatch.setattr(B, "measure_block", fake_block)
    monkeypatch.setattr(B, "gpu_state", lambda *a, **k: {"available": False})
    return B, calls


def test_bench_pair_alternates_and_retries(monkeypatch):
    import itertools
    # the candidate's 6th block is 20% slow -> cross-block guard -> retry
    cand = iter([8.0] * 5 + [9.6] + [8.0] * 20)
    B, calls = _patch_engine(monkeypatch, {"a": itertools.repeat(10.0), "b": cand})
    rec = B.bench_pair(_FakeOp(), _FakeExt(), "a", "b", 64, 128, rounds=9)
    assert calls[:4] == ["a", "b", "b", "a"]              # order alternates
    assert rec["valid_rounds"] == 9 and rec["invalid_crossblock_rounds"] == 0
    r6 = rec["rounds"][5]
    assert r6["retries"] == 1 and r6["valid"]               # retried once
    assert sum(r["retries"] for r in rec["rounds"]) == 1
    assert rec["median_speedup"] == 1.25 and rec["faster_rounds"] == "9/9"
    dec, _ = D.decide_v2(True, rec["valid_rounds"], rec["speedups"],
                         rec["bootstrap_ci_95"])
    assert dec == D.KEEP and not rec["filter_sensitive"]
    assert rec["algorithmic_bw_gbps_candidate"] == round(1e6 / 8e-6 / 1e9, 1)
    assert rec["harness"] == "paired-streaming-v2.3" and rec["caliber"] == "native"


def test_bench_pair_refuses_quarantined_and_unknown(monkeypatch):
    import itertools
    B, _ = _patch_engine(monkeypatch, {"a": itertools.repeat(1.0)})
    with pytest.raises(ValueError, match="quarantined"):
        B.bench_pair(_FakeOp(), _FakeExt(), "a", "q", 1, 1)
    with pytest.raises(ValueError, match="unknown variant"):
        B.bench_pair(_FakeOp(), _FakeExt(), "a", "zz", 1, 1)
    with pytest.raises(ValueError, match="cache mode"):
        B.bench_pair(_FakeOp(), _FakeExt(), "a", "b", 1, 1, mode="lukewarm")


def test_bench_matrix_rotates_and_classifies(monkeypatch):
    import itertools
    B, calls = _patch_engine(monkeypatch, {"a": itertools.repeat(10.0),
                                           "b": itertools.repeat(9.0),
                                           "alias_of_a": itertools.repeat(10.0),
                                           "c": itertools.repeat(12.0)})
    rec = B.bench_matrix(_FakeOp(), _FakeExt(), ["a", "b", "c"], 64, 128, rounds=6)
    assert calls[:9] == ["a", "b", "c", "b", "c", "a", "c", "a", "b"]
    assert rec["valid_rounds"] == 6
    assert rec["per_variant"]["b"]["median_us"] == 9.0
    [cell] = B.analyze_shape_winners([rec])
    assert (cell["winner"], cell["runner_up"]) == ("b", "a")
    assert cell["status"] == E.SIGNIFICANT_WINNER
    B.bench_matrix(_FakeOp(), _FakeExt(), ["alias_of_a", "b"], 1, 1, rounds=1)


# ------------------------------------------------------ negative-case runner
def test_negative_runner_records_and_pass_rule():
    from cudalab_amd.evaluator import negative as N

    def boom(msg):
        def f():
            raise RuntimeError(msg + "\nsecond line")
        return f

    ok = lambda: True      # noqa: E731
    bad = lambda: False    # noqa: E731
    r = N.run_case("v", "d", boom("x 必须是 2 维"), "reject", "必须是 2 维", ok)
    assert r["status"] == "rejected" and r["msg_match"] is True and r["pass"]
    assert r["exception_type"] == "RuntimeError" and r["message"] == "x 必须是 2 维"
    r = N.run_case("v", "d", boom("other"), "reject", "必须是 2 维", ok)
    assert r["msg_match"] is False and not r["pass"]
    r = N.run_case("v", "d", boom("anything"), "reject", None, ok)
    assert r["msg_match"] is None and r["pass"]
    r = N.run_case("v", "d", lambda: None, "reject", None, ok)
    assert r["status"] == "passed_without_exception" and not r["pass"]
    r = N.run_case("v", "d", lambda: None, "pass", None, ok)
    assert r["pass"] and r["post_check_ok"] is True
    r = N.run_case("v", "d", boom("x"), "pass", None, ok)
    assert not r["pass"]
    r = N.run_case("v", "d", boom("x 必须是 2 维"), "reject", "必须是 2 维", bad)
    assert r["post_check_ok"] is False and not r["pass"]
    r = N.run_case("v", "d", boom("y" * 400), "reject", None, ok)
    assert len(r["message"]) == 300
    s = N.run_case("v", "d", lambda: None, "skip", None, bad)
    assert s["status"] == "skipped" and "pass" not in s and s["post_check_ok"] is None
    recs = [N.run_case("v", "d", boom("m"), "reject", "m", ok),
            N.run_case("v", "d", lambda: None, "reject", None, ok),
            N.run_case("v", "d", lambda: None, "pass", None, ok), s]
    summ = N.summarize_cases(recs)
    assert summ == {"n_total": 4, "n_reject_expected": 2, "n_reject_ok": 1,
                    "n_pass_expected": 1, "n_pass_ok": 1, "n_skipped": 1,
                    "n_passed": 2, "all_pass": False}
    assert N.summarize_cases(recs[:1] + recs[2:])["all_pass"]


def test_timeline_summary_of_known_stamps():
    """The timeline's reduction on hand-made stamps (100 ticks per us):
    per launch, each point's median and maximum over the waves from the
    launch's first wave start; the span to its last y store; the gap to the
    next launch's first start; medians over the launches kept."""
    import numpy as np
    from cudalab_amd.evaluator.timeline import POINTS, summarize
    base = np.array([[0, 100, 150, 160, 170],      # wave 0 (ticks)
                     [20, 110, 200, 230, 250],     # wave 1
                     [40, 120, 210, 240, 260]])    # wave 2
    L = 3
    a = np.zeros((L, 3, 8), dtype=np.int64)
    for i in range(L):
        a[i, :, :5] = base + 1000 + i * 400        # launches 400 ticks apart
    s = summarize(a, 100.0, skip=0.0)
    assert s["launches_used"] == 2                 # the last launch has no successor
    p = s["points"]
    assert p[POINTS[0]] == {"p50_us": 0.2, "max_us": 0.4}
    assert p[POINTS[1]] == {"p50_us": 1.1, "max_us": 1.2}
    assert p[POINTS[2]] == {"p50_us": 2.0, "max_us": 2.1}
    assert p[POINTS[4]] == {"p50_us": 2.5, "max_us": 2.6}
    assert s["span_us"] == pytest.approx(2.6)
    assert s["gap_us"] == pytest.approx(4.0 - 2.6)


def test_floor_fit_recovers_a_line():
    """floor.fit_line: least squares t = t0 + bytes / B over the sizes from
    8 MiB up recovers the line that generated the points (and ignores the
    small sizes, where the launch floor dominates)."""
    from cudalab_amd.evaluator.floor import fit_line
    rows = [{"bytes": b, "us_per_launch": 1.25 + b / 6500e3}
            for b in (8 << 20, 16 << 20, 64 << 20, 256 << 20)]
    rows.append({"bytes": 1 << 20, "us_per_launch": 1.8})   # below the fit range
    fit = fit_line(rows)
    assert fit["points"] == 4
    assert abs(fit["t0_us"] - 1.25) < 1e-3
    assert abs(fit["GBps"] - 6500.0) < 0.5


def test_counter_report_derives_ratios():
    """counters.derived: the ratios the occupancy/latency/stall report prints
    come from the right counter pairs."""
    from cudalab_amd.evaluator.counters import derived, table
    c = {"MeanOccupancyPerCU": 4.5, "VmemLatency": 1800.0, "LdsLatency": 60.0,
         "LdsUtil": 7.0, "TCP_TCC_READ_REQ_LATENCY": 3000.0, "TCP_TCC_READ_REQ": 3.0,
         "SQ_WAIT_INST_LDS": 10.0, "SQ_WAIT_INST_ANY": 40.0,
         "TA_ADDR_STALLED_BY_TC_CYCLES": 5.0, "TA_TA_BUSY": 20.0,
         "TD_TC_STALL": 3.0, "TD_TD_BUSY": 12.0, "SQ_INSTS_VALU": 800.0,
         "SQ_INSTS_VMEM_RD": 60.0, "SQ_WAVES": 4.0,
         "_kernel": "void cq::(anonymous namespace)::int4gemv_lds_kernel<64, 6, 1, 512>(x)"}
    d = derived(c)
    assert d["l2_lat"] == 1000.0 and d["wait_lds"] == 0.25
    assert d["ta_tc"] == 0.25 and d["td_tc"] == 0.25
    assert d["valu_per_wave"] == 200.0 and d["vmem_per_wave"] == 15.0
    t = table([("int4", "4096x11008", c)])
    assert "int4gemv_lds_kernel<64, 6, 1, 512>" in t and "1800" in t


def test_window_prefilled_needs_the_wait_to_outlast_the_enqueue_with_margin():
    from cudalab_amd.ext import PREFILL_MARGIN_US, prefill_delay_us, window_prefilled
    d = prefill_delay_us(2000)
    assert window_prefilled(d, 3.0 * 2000)              # 3 us per launch: covered
    assert not window_prefilled(d, d)                    # enqueue as long as the wait
    assert not window_prefilled(d, d - PREFILL_MARGIN_US)  # inside the margin
    assert window_prefilled(d, d - PREFILL_MARGIN_US - 1.0)
    assert not window_prefilled(0.0, 0.0)                # no wait: never pre-filled
    # the default wait leaves the margin for 20-launch windows at 8 us per launch
    assert window_prefilled(prefill_delay_us(20), 8.0 * 20)


def test_timeline_by_workgroup_ranks_workgroups_sharing_a_cu():
    """Two workgroups of 2 waves on each of 16 CUs (logical blocks 4x..4x+3
    run on XCD x; blocks 4x, 4x+2 share one CU and 4x+1, 4x+3 another): the
    one that starts later on its CU passes its barrier later; by_workgroup
    must see it, keying a CU by its XCD and hardware id (the XCD map must
    invert the kernels' XCD-contiguous block mapping)."""
    import numpy as np
    from cudalab_amd.evaluator.timeline import by_workgroup, xcd_of_logical_block
    assert list(xcd_of_logical_block(16)) == [x for x in range(8) for _ in range(2)]
    assert list(xcd_of_logical_block(10)) == [0, 0, 1, 1, 2, 3, 4, 5, 6, 7]
    grid, wpg, tpu = 32, 2, 100.0
    a = np.zeros((3, grid * wpg, 8), dtype=np.int64)
    for wg in range(grid):
        cu, second = wg % 2, wg % 4 >= 2        # hardware ids repeat across XCDs
        for w in range(wpg):
            row = a[:, wg * wpg + w]
            row[:, 0] = 1000 + (20 if second else 0) + w          # start: +0.2 us
            row[:, 1] = 1000 + (150 if second else 90) + 5 * w    # barrier
            row[:, 5] = cu
    g = by_workgroup(a, tpu, wpg, skip=0.0)
    assert g["workgroups"] == grid and g["launches_used"] == 3
    assert g["barrier_first_on_cu_us"] == pytest.approx(0.95)    # (90 + 5) ticks
    assert g["barrier_second_on_cu_us"] == pytest.approx(1.55)   # (150 + 5) ticks
    assert len(g["barrier_by_xcd_us"]) == 8
    assert g["corr_start_barrier"] > 0.99
    with pytest.raises(ValueError):
        by_workgroup(a[:, :63], tpu, wpg)


def test_timeline_by_workgroup_constant_starts_give_nan_correlation():
    import math
    import numpy as np
    from cudalab_amd.evaluator.timeline import by_workgroup
    a = np.zeros((2, 4, 8), dtype=np.int64)
    a[:, :, 0] = 1000
    a[:, :, 1] = 1100
    a[:, :, 5] = np.arange(4)
    g = by_workgroup(a, 100.0, 1, skip=0.0)
    assert g["barrier_first_on_cu_us"] == pytest.approx(1.0)
    assert g["barrier_second_on_cu_us"] is None
    assert math.isnan(g["corr_start_barrier"])
