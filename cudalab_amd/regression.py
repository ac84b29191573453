"""Regression over every normal variant of the three GEMV operators.

Restates `scripts/regression_v07.py:37-80`:

* for int4gemv, gemv and qgemv, every variant of `variants()` (the
  quarantined ones are not run) goes through its correctness suite and its
  negative suite, with their records written under OUT/<op>/;
* a quarantine audit records, per operator, the three registry lists
  (`variants()`, `all_variants()`, `quarantined_variants()`) and whether a
  quarantined name leaked into the normal list;
* OUT/summary.json holds the per-variant results, OUT/quarantine_audit.json
  the audit.  The last line printed is "SUMMARY all_pass" or
  "SUMMARY FAILED: [...]", and the exit status is 0 or 1 to match.

Usage: python -m cudalab_amd.regression [--out DIR] [--ops int4gemv,qgemv]
The default OUT is experiments/regression/mi355x/ under the repository.
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
OPS = ("int4gemv", "gemv", "qgemv")


def run(out: Path, ops=OPS) -> dict:
    from .operators import get
    summary: dict = {"ops": {}, "quarantine": {}}
    for name in ops:
        op = get(name)
        ext = op.build()
        out_dir = out / name
        out_dir.mkdir(parents=True, exist_ok=True)
        normal = op.variants(ext)
        per_variant = {}
        ok_all = True
        for v in normal:
            c = op.run_correctness(ext, v, out_dir=out_dir)
            n = op.run_negative(ext, v, out_dir=out_dir)
            c_ok = bool(c.get("all_pass"))
            n_ok = bool(n.get("summary", {}).get("all_pass"))
            ok_all = ok_all and c_ok and n_ok
            per_variant[v] = {
                "correctness_all_pass": c_ok,
                "correctness_n_pass": c.get("summary", {}).get("n_pass"),
                "negative_all_pass": n_ok,
                "negative_n_passed": n.get("summary", {}).get("n_passed"),
            }
            print(f"[{name}] {v}: correctness={c_ok} "
                  f"({per_variant[v]['correctness_n_pass']}), negative={n_ok} "
                  f"({per_variant[v]['negative_n_passed']})", flush=True)
        quarantined = op.unsafe_variants(ext)
        summary["ops"][name] = {
            "variants_run": per_variant,
            "all_pass": ok_all,
            "quarantine_leaked_into_normal": [v for v in quarantined if v in normal],
        }
        summary["quarantine"][name] = {
            "variants()": normal,
            "all_variants()": ext.all_variants(),
            "quarantined_variants()": quarantined,
        }
    out.mkdir(parents=True, exist_ok=True)
    (out / "quarantine_audit.json").write_text(
        json.dumps(summary["quarantine"], indent=2))
    (out / "summary.json").write_text(json.dumps(summary["ops"], indent=2))
    return summary


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", type=Path,
                    default=ROOT / "experiments" / "regression" / "mi355x")
    ap.add_argument("--ops", default=",".join(OPS))
    a = ap.parse_args(argv)
    from . import _capi
    print(f"library: {_capi.version()}", flush=True)   # the build that ran
    ops = tuple(o for o in a.ops.split(",") if o)
    if not ops or any(o not in OPS for o in ops):
        print(f"regression: --ops must name some of {OPS}", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("regression: no GPU visible", file=sys.stderr)
        return 1
    summary = run(a.out, ops)
    bad = [k for k, d in summary["ops"].items()
           if not d["all_pass"] or d["quarantine_leaked_into_normal"]]
    print("SUMMARY all_pass" if not bad else f"SUMMARY FAILED: {bad}", flush=True)
    return 0 if not bad else 1


if __name__ == "__main__":
    sys.exit(main())
