"""Command line of the GEMV path: test, benchmark, profile, pytorch context
and one optimisation experiment, for the int4gemv, qgemv and gemv
operators on one MI355X.

Restates the commands of the reference's unified CLI for these operators
(`scripts/cudalab.py:109-415`; the same subcommands, option names and exit
codes, with --M / --H meaning N / K as there):

  test OP --variant V             correctness suite + negative suite
  benchmark pair OP --parent P --candidate C --M N --H K --tag T
  benchmark matrix OP --variants A,B,... --M N --H K --tag T
  benchmark full OP [--variants ...] --tag T     every bench shape x mode
  benchmark winners OP --tag T    per-cell winners of saved matrix records
  profile OP [--variants ...] --M N --H K        rocprofv3 kernel profile
  pytorch OP --M N --H K          framework context (torch.mv), no decision
  optimize OP --id ID --parent P --candidate C --hypothesis .. --changes ..
                                  correctness + negative + paired bench ->
                                  fixed decision rules -> experiment record
                                  (failed experiments are saved too)

Exit codes: 0 done (test: everything passed), 1 a suite failed, 2 a
variant was unknown or quarantined (nothing ran).

Differences forced by the platform: the profiler is rocprofv3 (one kernel
trace plus optional counter passes, `--counters`); the reference's NCU
cache-control and clock-control runs have no rocprofv3 counterpart, so
`--clock-control` is accepted and recorded only.  Benchmarks take the
timing caliber (`--caliber native|api`, default native) of this build's
engine.
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

OPS = ("int4gemv", "qgemv", "gemv")


def _dtype(s: str):
    import torch
    return {"float16": torch.float16, "float32": torch.float32}[s]


def _gate(op, ext, v: str) -> str | None:
    """None for a dispatchable variant (or a reference name accepted as its
    alias); the refusal message for an unknown or quarantined one (the
    reference's gate, scripts/cudalab.py:59-70 and the unknown-variant
    message of :121-123)."""
    avail = op.variants(ext)
    if v in avail or v in ext.aliases():
        return None
    if v in op.unsafe_variants(ext):
        return (f"变体 {v!r} 已被隔离（UNSAFE_HISTORICAL_EXPERIMENT / "
                f"REJECTED / NOT_FOR_NORMAL_DISPATCH），不能进入正常测试 / "
                f"基准 / 剖析路径 (variant {v!r} is quarantined and cannot "
                f"be tested, benchmarked or profiled)")
    return f"未知变体 {v!r}; 可用: {avail}"


def _print_pair(rec: dict) -> None:
    print(f"[pair] {rec['parent']} vs {rec['candidate']} "
          f"M={rec['shape'][0]} H={rec['shape'][1]} {rec['dtype']} "
          f"mode={rec['cache_mode']} caliber={rec['caliber']}")
    print(f"  valid rounds: {rec['valid_rounds']}/{rec['n_rounds']} "
          f"(invalid env: {rec['invalid_environment_rounds']})")
    print(f"  parent    median: {rec['parent_median_us']} us   algo BW: "
          f"{rec['algorithmic_bw_gbps_parent']} GB/s")
    print(f"  candidate median: {rec['candidate_median_us']} us   algo BW: "
          f"{rec['algorithmic_bw_gbps_candidate']} GB/s")
    print(f"  median speedup (parent/cand): {rec['median_speedup']}  "
          f"CI95: {rec['bootstrap_ci_95']}  faster rounds: {rec['faster_rounds']}")
    print(f"  raw_speedup: {rec['raw_speedup']}  (parent "
          f"{rec['raw']['parent_median_us']} us / candidate "
          f"{rec['raw']['candidate_median_us']} us)  CI95: "
          f"{rec['raw']['bootstrap_ci_95']}")
    print(f"  filtered_speedup: {rec['filtered_speedup']}  CI95: "
          f"{rec['filtered']['bootstrap_ci_95']}")
    print(f"  filter_sensitive: {rec['filter_sensitive']} -- "
          f"{rec['filter_sensitive_reason']}")
    print(f"  rejected_samples: {rec['rejected_samples']}")


def _print_matrix(rec: dict) -> None:
    print(f"[matrix] M={rec['shape'][0]} H={rec['shape'][1]} {rec['dtype']} "
          f"mode={rec['cache_mode']} caliber={rec['caliber']} valid "
          f"{rec['valid_rounds']}/{rec['n_rounds']} rounds")
    for v in rec["variants"]:
        pv = rec["per_variant"][v]
        print(f"  {v:<22} median {pv['median_us']} us   algo BW "
              f"{pv['algorithmic_bw_gbps']} GB/s")


def _print_winner(w: dict) -> None:
    print(f"M={w['shape'][0]:<5} H={w['shape'][1]:<5} {w['dtype']:<8} "
          f"{w['cache_mode']:<10} winner={w['winner']} "
          f"runner_up={w['runner_up']} ratio={w['median_ratio']} "
          f"CI95={w['bootstrap_ci_95']} stat={w['statistical_relation']} "
          f"policy={w['policy_decision']} status={w['status']}")


# ---- test --------------------------------------------------------------------

def cmd_test(a) -> int:
    from .operators import get
    op = get(a.op)
    ext = op.build()
    msg = _gate(op, ext, a.variant)
    if msg:
        print(msg, file=sys.stderr)
        return 2
    res = op.run_correctness(ext, a.variant,
                             out_dir=Path(a.out_dir) if a.out_dir else None)
    s = res["summary"]
    print(f"[correctness] {a.variant}: all_pass={res['all_pass']} "
          f"n_pass={s['n_pass']}/{s['n_total']} "
          f"max_abs={s['max_abs_error']} max_rel={s['max_rel_error']}")
    print(f"  -> {res['saved']}")
    neg = op.run_negative(ext, a.variant,
                          out_dir=Path(a.neg_out_dir) if a.neg_out_dir else None)
    n = neg["summary"]
    print(f"[negative] all_pass={n['all_pass']} "
          f"n_passed={n['n_passed']}/{n['n_total']} "
          f"(reject_ok={n['n_reject_ok']}/{n['n_reject_expected']}, "
          f"pass_ok={n['n_pass_ok']}/{n['n_pass_expected']}, "
          f"skipped={n['n_skipped']})")
    return 0 if (res["all_pass"] and n["all_pass"]) else 1


# ---- benchmark -----------------------------------------------------------------

def _bench_out(op, a) -> Path:
    return Path(a.out_dir) if getattr(a, "out_dir", None) else op.bench_dir


def cmd_bench_pair(a) -> int:
    from .evaluator.bench import bench_pair, save_record
    from .operators import get
    op = get(a.op)
    ext = op.build()
    for v in (a.parent, a.candidate):
        msg = _gate(op, ext, v)
        if msg:
            print(msg, file=sys.stderr)
            return 2
    rec = bench_pair(op, ext, a.parent, a.candidate, a.M, a.H, _dtype(a.dtype),
                     mode=a.mode, rounds=a.rounds, caliber=a.caliber)
    p = save_record(rec, _bench_out(op, a), a.tag)
    _print_pair(rec)
    print(f"saved -> {p}")
    return 0


def cmd_bench_matrix(a) -> int:
    from .evaluator.bench import bench_matrix, save_record
    from .operators import get
    op = get(a.op)
    ext = op.build()
    variants = [v.strip() for v in a.variants.split(",") if v.strip()]
    for v in variants:
        msg = _gate(op, ext, v)
        if msg:
            print(msg, file=sys.stderr)
            return 2
    rec = bench_matrix(op, ext, variants, a.M, a.H, _dtype(a.dtype),
                       mode=a.mode, rounds=a.rounds, caliber=a.caliber)
    p = save_record(rec, _bench_out(op, a), a.tag)
    _print_matrix(rec)
    print(f"saved -> {p}")
    return 0


def cmd_bench_full(a) -> int:
    """Every bench shape x dtype x {hot, streaming} as a matrix, then the
    per-cell winners (scripts/cudalab.py:163-186)."""
    from .evaluator.bench import (HARNESS_VERSION, analyze_shape_winners,
                                  bench_matrix, save_record)
    from .operators import get
    op = get(a.op)
    ext = op.build()
    variants = ([v.strip() for v in a.variants.split(",") if v.strip()]
                if a.variants else op.variants(ext))
    for v in variants:
        msg = _gate(op, ext, v)
        if msg:
            print(msg, file=sys.stderr)
            return 2
    out = _bench_out(op, a)
    records = []
    for (M, H) in op.bench_shapes:
        for dtype_name in op.dtypes:
            for mode in ("hot", "streaming"):
                tag = f"{a.tag}_M{M}_H{H}_{dtype_name}_{mode}"
                print(f"=== {tag} ===", flush=True)
                rec = bench_matrix(op, ext, variants, M, H, _dtype(dtype_name),
                                   mode=mode, rounds=a.rounds, caliber=a.caliber)
                save_record(rec, out, tag)
                _print_matrix(rec)
                records.append(rec)
    winners = analyze_shape_winners(records)
    wp = save_record({"harness": HARNESS_VERSION, "operator": op.name,
                      "shape_winners": winners}, out, f"{a.tag}_shape_winners")
    for w in winners:
        _print_winner(w)
    print(f"shape winners -> {wp}")
    return 0


def cmd_bench_winners(a) -> int:
    """Per-cell winners of the matrix records saved under one tag
    (scripts/cudalab.py:189-209).  CPU only."""
    from .evaluator.bench import analyze_shape_winners
    from .operators import get
    op = get(a.op)
    out = _bench_out(op, a)
    recs = []
    for p in sorted(out.glob(f"{a.tag}_M*_H*.json")):
        r = json.loads(p.read_text())
        if "per_variant" in r:
            recs.append(r)
    winners = analyze_shape_winners(recs)
    path = out / f"{a.tag}_shape_winners.json"
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps({"operator": op.name, "shape_winners": winners},
                               indent=2, ensure_ascii=False))
    for w in winners:
        _print_winner(w)
    print(f"saved -> {path}")
    return 0


# ---- profile ---------------------------------------------------------------------

def _counter_groups(spec: str | None) -> list[list[str]]:
    """"A,B;C" -> [["A", "B"], ["C"]]: one rocprofv3 --pmc pass per group."""
    if not spec:
        return []
    return [[c.strip() for c in g.split(",") if c.strip()]
            for g in spec.split(";") if g.strip()]


def cmd_profile(a) -> int:
    from .evaluator.profiler import profile_variant
    from .operators import get
    op = get(a.op)
    ext = op.build()
    variants = ([v.strip() for v in a.variants.split(",") if v.strip()]
                if a.variants else op.variants(ext))
    for v in variants:
        msg = _gate(op, ext, v)
        if msg:
            print(msg, file=sys.stderr)
            return 2
    base = Path(a.out_dir) if a.out_dir else op.profiles_dir / "runs"
    groups = _counter_groups(a.counters)
    for v in variants:
        out = base / f"{v}_M{a.M}_H{a.H}"
        print(f"== profiling {v} ==", flush=True)
        s = profile_variant(op, v, a.M, a.H, out_dir=out, counters=groups)
        s["clock_control"] = {"requested": a.clock_control,
                              "applied": False,
                              "note": "rocprofv3 does not lock clocks"}
        (out / "summary.json").write_text(json.dumps(s, indent=2))
        if s["errors"]:
            print(f"   ERROR: {'; '.join(s['errors'])[:300]}", file=sys.stderr)
        print(f"   duration={s['kernel_duration_us']}us "
              f"algo_bw={s['algorithmic_bw_gbps']}GB/s "
              f"counters={s['counters']} -> {out / 'summary.json'}")
    return 0


# ---- pytorch context -----------------------------------------------------------------

def cmd_pytorch(a) -> int:
    from .operators import get
    op = get(a.op)
    d = op.pytorch_ref_latency(a.M, a.H, _dtype(a.dtype))
    print(json.dumps(d, indent=2, ensure_ascii=False))
    return 0


# ---- optimize ----------------------------------------------------------------------

def cmd_optimize(a) -> int:
    """One optimisation experiment (scripts/cudalab.py:224-331): the
    candidate's correctness and negative suites, a paired benchmark
    against the parent, the fixed decision rules with the filter gate, an
    optional profile, and one experiment record saved whatever the
    outcome."""
    from .evaluator.bench import bench_pair, save_record
    from .evaluator.decision import (apply_filter_gate, decide_v2,
                                     statistical_relation)
    from .evaluator.experiment import save_experiment
    from .operators import get
    op = get(a.op)
    ext = op.build()
    for v in (a.parent, a.candidate):
        msg = _gate(op, ext, v)
        if msg:
            print(msg, file=sys.stderr)
            return 2

    print(f"== [{a.id}] correctness: {a.candidate} ==", flush=True)
    corr = op.run_correctness(ext, a.candidate)
    print(f"   all_pass={corr['all_pass']} -> {corr['saved']}")
    print(f"== [{a.id}] negative suite: {a.candidate} ==", flush=True)
    neg = op.run_negative(ext, a.candidate)["summary"]
    print(f"   all_pass={neg['all_pass']} ({neg['n_passed']}/{neg['n_total']})")

    print(f"== [{a.id}] paired bench: {a.parent} vs {a.candidate} "
          f"({a.M},{a.H}) {a.dtype} {a.mode} ==", flush=True)
    tag = f"{a.id}_pair_{a.parent}_vs_{a.candidate}_M{a.M}_H{a.H}_{a.dtype}_{a.mode}"
    paired = bench_pair(op, ext, a.parent, a.candidate, a.M, a.H, _dtype(a.dtype),
                        mode=a.mode, rounds=a.rounds, caliber=a.caliber)
    bp = save_record(paired, op.bench_dir, tag)
    _print_pair(paired)

    decision, detail = decide_v2(corr["all_pass"] and neg["all_pass"],
                                 paired["valid_rounds"], paired["speedups"],
                                 paired["bootstrap_ci_95"])
    decision, detail = apply_filter_gate(decision, detail,
                                         paired["filter_sensitive"],
                                         paired["filter_sensitive_reason"])
    rel = statistical_relation(paired["bootstrap_ci_95"])
    detail["statistical_relation"] = rel
    detail["policy_decision"] = decision
    print(f"== [{a.id}] decision: {decision} ==")
    print(f"   {detail.get('rule')}")
    print(f"   statistical_relation: {rel} (from the CI95 alone, independent "
          "of the 5% policy band)")
    print(f"   policy_decision: {decision} (acceptance policy, after the "
          "filter gate)")

    profile_obs = None
    if a.profile:
        from .evaluator.profiler import profile_variant
        out = op.profiles_dir / "runs" / f"{a.candidate}_M{a.M}_H{a.H}"
        s = profile_variant(op, a.candidate, a.M, a.H, out_dir=out)
        profile_obs = {"file": str(out / "summary.json"),
                       "kernel_duration_us": s.get("kernel_duration_us"),
                       "algorithmic_bw_gbps": s.get("algorithmic_bw_gbps"),
                       "errors": s.get("errors")}
        print(f"   profile -> {out / 'summary.json'}")

    record = {
        "id": a.id,
        "operator": op.name,
        "parent": a.parent,
        "candidate": a.candidate,
        "hypothesis": a.hypothesis,
        "changes": a.changes,
        "correctness": corr,
        "negative": neg,
        "paired_benchmark": {
            "file": str(bp),
            "harness": paired["harness"],
            "caliber": paired["caliber"],
            "shape": [a.M, a.H], "dtype": a.dtype, "cache_mode": a.mode,
            "parent": a.parent, "candidate": a.candidate,
            "paired_rounds": paired["n_rounds"],
            "valid_rounds": paired["valid_rounds"],
            "invalid_environment_rounds": paired["invalid_environment_rounds"],
            "invalid_dvfs_rounds": paired["invalid_dvfs_rounds"],
            "median_speedup_parent_over_candidate": paired["median_speedup"],
            "bootstrap_ci_95": paired["bootstrap_ci_95"],
            "faster_rounds_candidate": paired["faster_rounds"],
            "parent_median_us": paired["parent_median_us"],
            "candidate_median_us": paired["candidate_median_us"],
            "raw_speedup": paired["raw_speedup"],
            "filtered_speedup": paired["filtered_speedup"],
            "filter_sensitive": paired["filter_sensitive"],
            "filter_sensitive_reason": paired["filter_sensitive_reason"],
            "rejected_samples": paired["rejected_samples"],
        },
        "profile_observation": profile_obs,
        "decision": detail,
    }
    p = save_experiment(record, op.experiments_dir, op.experiment_prefix())
    print(f"experiment record -> {p}")
    return 0


# ---- parser ---------------------------------------------------------------------------

def build_parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(prog="python -m cudalab_amd.cli",
                                 description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)

    p = sub.add_parser("test", help="correctness suite + negative suite")
    p.add_argument("op", choices=OPS)
    p.add_argument("--variant", required=True)
    p.add_argument("--out-dir", default=None)
    p.add_argument("--neg-out-dir", default=None)
    p.set_defaults(fn=cmd_test)

    pb = sub.add_parser("benchmark", help="paired benchmark engine")
    bsub = pb.add_subparsers(dest="bcmd", required=True)

    def common(q, tag_required=True):
        q.add_argument("--dtype", default="float16", choices=["float16", "float32"])
        q.add_argument("--mode", default="streaming",
                       choices=["hot", "streaming", "x-rotate"])
        q.add_argument("--rounds", type=int, default=9)
        q.add_argument("--caliber", default="native", choices=["native", "api"])
        q.add_argument("--tag", required=tag_required)
        q.add_argument("--out-dir", default=None)

    q = bsub.add_parser("pair")
    q.add_argument("op", choices=OPS)
    q.add_argument("--parent", required=True)
    q.add_argument("--candidate", required=True)
    q.add_argument("--M", type=int, required=True)
    q.add_argument("--H", type=int, required=True)
    common(q)
    q.set_defaults(fn=cmd_bench_pair)

    q = bsub.add_parser("matrix")
    q.add_argument("op", choices=OPS)
    q.add_argument("--variants", required=True)
    q.add_argument("--M", type=int, required=True)
    q.add_argument("--H", type=int, required=True)
    common(q)
    q.set_defaults(fn=cmd_bench_matrix)

    q = bsub.add_parser("full")
    q.add_argument("op", choices=OPS)
    q.add_argument("--variants", default=None)
    q.add_argument("--rounds", type=int, default=9)
    q.add_argument("--caliber", default="native", choices=["native", "api"])
    q.add_argument("--tag", required=True)
    q.add_argument("--out-dir", default=None)
    q.set_defaults(fn=cmd_bench_full)

    q = bsub.add_parser("winners")
    q.add_argument("op", choices=OPS)
    q.add_argument("--tag", required=True)
    q.add_argument("--out-dir", default=None)
    q.set_defaults(fn=cmd_bench_winners)

    p = sub.add_parser("profile", help="rocprofv3 kernel profile")
    p.add_argument("op", choices=OPS)
    p.add_argument("--variants", default=None)
    p.add_argument("--M", type=int, default=4096)
    p.add_argument("--H", type=int, default=4096)
    p.add_argument("--counters", default=None,
                   help='counter passes, e.g. "FETCH_SIZE;WRITE_SIZE" '
                        "(one rocprofv3 --pmc run per ;-separated group)")
    p.add_argument("--clock-control", default="base",
                   choices=["base", "none", "reset"])
    p.add_argument("--out-dir", default=None)
    p.set_defaults(fn=cmd_profile)

    p = sub.add_parser("pytorch", help="PyTorch context (no decision)")
    p.add_argument("op", choices=OPS)
    p.add_argument("--M", type=int, required=True)
    p.add_argument("--H", type=int, required=True)
    p.add_argument("--dtype", default="float16", choices=["float16", "float32"])
    p.set_defaults(fn=cmd_pytorch)

    p = sub.add_parser("optimize", help="one optimisation experiment")
    p.add_argument("op", choices=OPS)
    p.add_argument("--id", required=True)
    p.add_argument("--parent", required=True)
    p.add_argument("--candidate", required=True)
    p.add_argument("--hypothesis", required=True)
    p.add_argument("--changes", required=True)
    p.add_argument("--M", type=int, default=4096)
    p.add_argument("--H", type=int, default=4096)
    p.add_argument("--dtype", default="float16", choices=["float16", "float32"])
    p.add_argument("--mode", default="streaming",
                   choices=["hot", "streaming", "x-rotate"])
    p.add_argument("--rounds", type=int, default=9)
    p.add_argument("--caliber", default="native", choices=["native", "api"])
    p.add_argument("--profile", action="store_true")
    p.set_defaults(fn=cmd_optimize)
    return ap


def main(argv=None) -> int:
    a = build_parser().parse_args(argv)
    if not (a.cmd == "benchmark" and a.bcmd == "winners"):
        import torch
        if not torch.cuda.is_available():
            print("cudalab_amd.cli: no GPU visible", file=sys.stderr)
            return 1
    return a.fn(a)


if __name__ == "__main__":
    sys.exit(main())
