"""Three-generation native kernel-loop timing: FP16, INT8 and INT4 GEMV at
4096x4096 under the same harness.

Restates `scripts/gen3_native_timing.py:30-67`: each generation's variant
is timed with the extension's `native_timing` (back-to-back launches in
native code, HIP events per window of 64 launches, 10 windows), once after
200 and once after 5000 warm-up launches, on seeded inputs (seed 1234 for W
and x).  The reference's variant names are used (`gemv_vec4_row`,
`qgemv_vec16_row`, `int4gemv_rowtile4_hx`); this build accepts them as
aliases of its CDNA4 incumbents.  One JSON document per generation is
written to OUT/<op>/native_timing_<variant>_4096.json and the medians are
printed.

This is the hot caliber of the reference (one W resident across all
launches); the HBM-cold comparison is the streaming sweep
(`python -m cudalab_amd.evaluator.sweep`).

Usage: python -m cudalab_amd.gen3 [--out DIR] [--n 4096] [--k 4096]
The default OUT is experiments/ under the repository.
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HARNESS = ("native kernel-loop: continuous raw launches in native code, "
           "HIP events / 64, 10 windows")
NOTE = ("native kernel-loop caliber: launches back to back in native code, "
        "HIP events / N; excludes the Python boundary (unlike the bench "
        "engine's API caliber) and is not a per-dispatch profiler duration")
SEED = 1234
GENERATIONS = (("gemv", "gemv_vec4_row"), ("qgemv", "qgemv_vec16_row"),
               ("int4gemv", "int4gemv_rowtile4_hx"))


def _inputs(op: str, N: int, K: int):
    import torch
    if op == "gemv":
        from .operators.gemv import make_w, make_x
        return (make_w(N, K, torch.float16, seed=SEED),
                make_x(K, torch.float16, seed=SEED))
    if op == "qgemv":
        from .operators.qgemv import make_w_q, make_x_q
        Wq, s, _W = make_w_q(N, K, seed=SEED)
        return Wq, s, make_x_q(K, seed=SEED)
    from .operators.int4gemv import make_w4, make_x4
    Wp, s, _W = make_w4(N, K, seed=SEED)
    return Wp, s, make_x4(K, seed=SEED)


def time_generation(op: str, variant: str, N: int, K: int) -> dict:
    import torch
    from .build import build
    ext = build(op)
    tensors = _inputs(op, N, K)
    out = torch.empty(N, dtype=torch.float16, device="cuda")
    res = {}
    for tag, warmup in (("w200", 200), ("w5000", 5000)):
        d = dict(ext.native_timing(variant, *tensors, out, warmup, 10, 64))
        d["note"] = NOTE
        res[tag] = d
    return {"variant": variant, "resolves_to": ext.resolve(variant),
            "shape": f"{N}x{K}x{K}", "harness": HARNESS, "windows": 10,
            "launches_per_window": 64, "seed": SEED,
            "w200": res["w200"], "w5000": res["w5000"]}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", type=Path, default=ROOT / "experiments")
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--k", type=int, default=4096)
    a = ap.parse_args(argv)
    from . import _capi
    print(f"library: {_capi.version()}", flush=True)   # the build that ran
    import torch
    if not torch.cuda.is_available():
        print("gen3: no GPU visible", file=sys.stderr)
        return 1
    for op, variant in GENERATIONS:
        doc = time_generation(op, variant, a.n, a.k)
        path = a.out / op / f"native_timing_{variant}_{a.n}.json"
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
        print(path)
        print(f"  {variant} -> {doc['resolves_to']}")
        print("  w200 median:", doc["w200"]["median_us"])
        print("  w5000 median:", doc["w5000"]["median_us"], flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
