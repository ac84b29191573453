"""Command line of the paired A/B methodology on one GPU.

  pair    parent vs candidate (bench_pair), the candidate's correctness
          suite first, then the fixed decision rules and the filter gate:
          one line with policy decision, statistical relation, median
          round speedup, CI95 and valid rounds
  matrix  several variants round-robin (bench_matrix), classified per
          cell (analyze_shape_winners)

This is how an incumbent is chosen: a candidate replaces the parent only
on KEEP (median >= 1.05, >= 70% of rounds faster, CI95 above 1.00, guards
not changing the conclusion, correctness passing).  Restates the decision
flow of the reference's optimisation command over
cudalab/evaluator/{bench,stats,decision,experiment}.py.

Usage:
  python -m cudalab_amd.evaluator.ab pair --op int4gemv \\
      --parent int4gemv_wave_r2 --candidate int4gemv_cdna4 --shape 4096 4096
  python -m cudalab_amd.evaluator.ab matrix --op int4gemv \\
      --variants int4gemv_cdna4,int4gemv_lds_r1,int4gemv_wave_r2 --shape 4096 4096
Options: --mode streaming|hot|x-rotate, --rounds, --iters, --batch,
--caliber native|api, --no-correctness, --out DIR (JSON records).
"""
from __future__ import annotations

import argparse
import sys
import tempfile
from pathlib import Path

from . import decision as D


def decide_pair(record: dict, correctness_pass: bool) -> dict:
    """Policy decision and statistical relation of a bench_pair record."""
    dec, detail = D.decide_v2(correctness_pass, record["valid_rounds"],
                              record["speedups"], record["bootstrap_ci_95"])
    dec, detail = D.apply_filter_gate(dec, detail, record["filter_sensitive"],
                                      record["filter_sensitive_reason"])
    return {"policy_decision": dec,
            "statistical_relation": D.statistical_relation(record["bootstrap_ci_95"]),
            "rule": detail.get("rule"),
            "correctness_pass": correctness_pass}


def _pair_line(rec: dict, verdict: dict) -> str:
    return (f"{rec['operator']} {rec['shape'][0]}x{rec['shape'][1]} {rec['cache_mode']} "
            f"{rec['caliber']}: {rec['candidate']} vs {rec['parent']}: "
            f"{verdict['policy_decision']} ({verdict['statistical_relation']}), "
            f"median speedup {rec['median_speedup']}, CI95 {rec['bootstrap_ci_95']}, "
            f"faster rounds {rec['faster_rounds']}, valid {rec['valid_rounds']}/"
            f"{rec['n_rounds']}, parent {rec['parent_median_us']} us "
            f"({rec['algorithmic_bw_gbps_parent']} GB/s), candidate "
            f"{rec['candidate_median_us']} us ({rec['algorithmic_bw_gbps_candidate']} GB/s)")


def _cell_line(rec: dict, cell: dict) -> str:
    meds = ", ".join(f"{v} {u}" for v, u in sorted(cell["all_variants_median_us"].items(),
                                                   key=lambda kv: kv[1]))
    return (f"{rec['operator']} {rec['shape'][0]}x{rec['shape'][1]} {rec['cache_mode']} "
            f"{rec['caliber']}: winner {cell['winner']} over {cell['runner_up']}: "
            f"{cell['status']} (policy {cell['policy_decision']}, "
            f"{cell['statistical_relation']}), ratio {cell['median_ratio']}, "
            f"CI95 {cell['bootstrap_ci_95']}, valid {cell['valid_rounds']}; "
            f"medians us: {meds}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    for name in ("pair", "matrix"):
        p = sub.add_parser(name)
        p.add_argument("--op", required=True, choices=("int4gemv", "qgemv", "gemv"))
        p.add_argument("--shape", type=int, nargs=2, required=True, metavar=("N", "K"))
        p.add_argument("--mode", default="streaming")
        p.add_argument("--rounds", type=int, default=9)
        p.add_argument("--iters", type=int, default=100)
        p.add_argument("--batch", type=int, default=32)
        p.add_argument("--caliber", default="native", choices=("native", "api"))
        p.add_argument("--out", type=Path, default=None)
        if name == "pair":
            p.add_argument("--parent", required=True)
            p.add_argument("--candidate", required=True)
            p.add_argument("--no-correctness", action="store_true")
        else:
            p.add_argument("--variants", required=True)
    a = ap.parse_args(argv)
    from .. import _capi
    print(f"library: {_capi.version()}", flush=True)   # the build that ran

    import torch
    if not torch.cuda.is_available():
        print("ab: no GPU visible", file=sys.stderr)
        return 1
    from ..operators import get
    from .bench import analyze_shape_winners, bench_matrix, bench_pair, save_record
    op = get(a.op)
    ext = op.build()
    N, K = a.shape
    if a.cmd == "pair":
        ok = True
        if not a.no_correctness:
            res = op.run_correctness(
                ext, a.candidate,
                out_dir=a.out or Path(tempfile.mkdtemp(prefix="cq_ab_")))
            ok = bool(res["all_pass"])
        rec = bench_pair(op, ext, a.parent, a.candidate, N, K, mode=a.mode,
                         rounds=a.rounds, iters=a.iters, batch=a.batch,
                         caliber=a.caliber)
        rec["verdict"] = decide_pair(rec, ok)
        print(_pair_line(rec, rec["verdict"]), flush=True)
        tag = f"pair_{a.candidate}_vs_{a.parent}_{N}x{K}_{a.mode}"
    else:
        variants = [v for v in a.variants.split(",") if v]
        rec = bench_matrix(op, ext, variants, N, K, mode=a.mode, rounds=a.rounds,
                           iters=a.iters, batch=a.batch, caliber=a.caliber)
        [cell] = analyze_shape_winners([rec])
        rec["cell"] = cell
        print(_cell_line(rec, cell), flush=True)
        tag = f"matrix_{a.op}_{N}x{K}_{a.mode}"
    if a.out:
        path = save_record(rec, a.out, tag)
        print(f"record: {path}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
