"""Shape sweep of the GEMV path on one GPU: µs per call, effective GB/s,
fraction of HBM peak and of the measured read ceiling, for the three
generations INT4, INT8 and FP16 over the reference's five bench shapes
(cudalab/operators/int4gemv.py:30-36 lists the same matrix) in streaming
(HBM-cold pool) and hot (one resident set) modes.

Timing caliber: the same as bench.py's headline -- untimed launches for at
least 100 ms, then K back-to-back launches on one stream between two HIP
events, queued behind an on-device wait so that the window times the GPU
and not the host's submission (cq_pool_timing).  The read ceiling is
cq_read_ceiling over an equally cold pool of the same bytes, same caliber.

Usage: python -m cudalab_amd.evaluator.sweep [--steps K] [--json FILE]
           [--ops int4gemv,qgemv,gemv] [--modes streaming,hot,misaligned]
           [--shapes NxK,NxK...] [--variant OP=V1,V2 ...]
Other shapes (e.g. Llama-70B's 8192x28672) and several variants per
operator (e.g. the incumbent against *_lds_tiled) time the same way.
"misaligned" is the streaming pool with W and x moved off their 16-byte
alignment (the scalar fallback, bit-identical to *_baseline).
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from ..ext import pool_timing, prefill_delay_us, read_ceiling
from ..build import build
from .bench import cold_pool_sets

HBM_PEAK_GBS = 8000.0
SHAPES = [(1024, 4096), (4096, 1024), (4096, 4096), (11008, 4096),
          (4096, 11008)]
OPS = {"int4gemv": "int4gemv_cdna4", "qgemv": "qgemv_cdna4",
       "gemv": "gemv_cdna4"}


def algorithmic_bytes(op: str, N: int, K: int) -> int:
    if op == "int4gemv":
        from ..operators.int4gemv import int4_bytes
        return int4_bytes(N, K)
    if op == "gemv":
        from ..operators.gemv import gemv_bytes
        return gemv_bytes(N, K, 2)
    from ..operators.qgemv import q8_bytes
    return q8_bytes(N, K)


MODES = ("streaming", "hot", "misaligned")


def offset_copy(t: torch.Tensor, offset_bytes: int) -> torch.Tensor:
    """The same values at a base address `offset_bytes` past a 16-byte
    boundary (a view into a slightly larger byte buffer)."""
    n = t.numel() * t.element_size()
    flat = torch.empty(n + 64, dtype=torch.uint8, device=t.device)
    view = flat[offset_bytes:offset_bytes + n].view(t.dtype).view_as(t)
    view.copy_(t)
    return view


def make_sets(op: str, N: int, K: int, mode: str, seed: int = 1234):
    """Input sets drawn on the device: a pool of more than 512 MiB of
    distinct sets for "streaming" and "misaligned", one set for "hot".
    INT4/INT8 sets are (W, scale, x, out); FP16 sets are (W, x, out).
    "misaligned" moves W one byte (INT4/INT8; two for FP16) and x two bytes
    off their 16-byte alignment (the offsets of the reference's fallback
    tests): every call then runs the scalar kernel, as the reference's did."""
    if op == "int4gemv":
        from ..operators.int4gemv import device_random_set
    elif op == "gemv":
        from ..operators.gemv import device_random_set
    else:
        from ..operators.qgemv import device_random_set
    if mode not in MODES:
        raise ValueError(f"unknown mode {mode!r} (one of {MODES})")
    nbytes = algorithmic_bytes(op, N, K)
    n = cold_pool_sets(nbytes) if mode != "hot" else 1
    sets = []
    for i in range(n):
        st = device_random_set(N, K, seed + 100000 + i)
        if mode == "misaligned":
            w_off = 2 if op == "gemv" else 1
            xi = 1 if op == "gemv" else 2
            st = tuple(offset_copy(t, w_off) if j == 0 else
                       offset_copy(t, 2) if j == xi else t
                       for j, t in enumerate(st))
        sets.append(st)
    return sets, nbytes


def window_us(op: str, variant: str, sets, steps: int, warmup: int) -> float:
    """µs per call of one pre-filled window; a window whose enqueue
    outlasted its on-device wait is timed again behind a wait twice the
    enqueue time."""
    torch.cuda.synchronize()
    r = pool_timing(op, variant, sets, warmup=warmup, n_launches=steps,
                    per_kernel=False, burn_ms=100.0,
                    delay_us=prefill_delay_us(steps))
    if not r["prefilled"]:
        r = pool_timing(op, variant, sets, warmup=0, n_launches=steps,
                        per_kernel=False,
                        delay_us=min(1e6, 2.0 * r["host_us"] + 500.0))
    torch.cuda.synchronize()
    return r["total_us"] / steps


def _record(op: str, ext, variant: str, N: int, K: int, mode: str,
            steps: int, warmup: int, ceiling: bool = True) -> dict:
    sets, nbytes = make_sets(op, N, K, mode)
    x0 = sets[0][1] if op == "gemv" else sets[0][2]
    plan = ext.describe(variant, sets[0][0], x0)
    us = window_us(op, variant, sets, steps, warmup)
    rec = {"op": op, "variant": variant, "N": N, "K": K, "mode": mode,
           "pool_sets": len(sets), "bytes_per_call": nbytes,
           "us_per_call": round(us, 4), "GBps": round(nbytes / us / 1e3, 1),
           "frac_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
           "plan": {k: plan[k] for k in ("kernel", "cw", "j", "r", "tile", "block", "grid")}}
    if mode == "streaming" and ceiling:
        c = read_ceiling(nbytes, warmup=warmup, n_launches=steps, burn_ms=100.0,
                         delay_us=prefill_delay_us(steps))
        rec["ceiling_us"] = round(c["us_per_call"], 4)
        rec["frac_ceiling"] = round(c["us_per_call"] / us, 4)
    del sets
    torch.cuda.empty_cache()
    return rec


def run(ops=tuple(OPS), shapes=SHAPES, modes=("streaming", "hot"),
        steps: int = 2000, warmup: int = 200,
        variants: dict | None = None, ceiling: bool = True) -> list[dict]:
    """One record per (op, variant, shape, mode); `variants` maps an op to
    the variants to time (default: its incumbent); `ceiling` False skips
    the read-ceiling measurement (profiling runs)."""
    out = []
    for op in ops:
        ext = build(op)
        for variant in (variants or {}).get(op, [OPS[op]]):
            for (N, K) in shapes:
                for mode in modes:
                    out.append(_record(op, ext, variant, N, K, mode, steps, warmup,
                                       ceiling))
    return out


def table(records: list[dict]) -> str:
    lines = [f"{'variant':<20} {'N':>6} {'K':>6} {'mode':<9} {'us/call':>8} "
             f"{'GB/s':>7} {'%peak':>6} {'ceil_us':>8} {'%ceil':>6}  plan"]
    for r in records:
        p = r["plan"]
        tile = f" tile={p['tile']}" if p.get("tile", "0") != "0" else ""
        plan = (f"{p['kernel']} cw={p['cw']} j={p['j']} r={p['r']}{tile} "
                f"block={p['block']} grid={p['grid']}")
        ceil = (f"{r['ceiling_us']:>8.3f} {100 * r['frac_ceiling']:>5.1f}%"
                if "ceiling_us" in r else f"{'-':>8} {'-':>6}")
        lines.append(f"{r['variant']:<20} {r['N']:>6} {r['K']:>6} {r['mode']:<9} "
                     f"{r['us_per_call']:>8.3f} {r['GBps']:>7.0f} "
                     f"{100 * r['frac_peak']:>5.1f}% {ceil}  {plan}")
    return "\n".join(lines)


def speedups(records: list[dict]) -> str:
    """INT4 vs INT8 vs FP16 per shape and mode (µs ratios)."""
    by = {(r["op"], r["N"], r["K"], r["mode"]): r["us_per_call"] for r in records
          if r["variant"] == OPS[r["op"]]}
    lines = [f"{'N':>6} {'K':>6} {'mode':<9} {'int4 us':>8} {'int8 us':>8} "
             f"{'fp16 us':>8} {'int8/int4':>9} {'fp16/int4':>9}"]
    for (op, N, K, mode), us in by.items():
        if op != "int4gemv":
            continue
        q8, f16 = by.get(("qgemv", N, K, mode)), by.get(("gemv", N, K, mode))
        if q8 is None or f16 is None:
            continue
        lines.append(f"{N:>6} {K:>6} {mode:<9} {us:>8.3f} {q8:>8.3f} {f16:>8.3f} "
                     f"{q8 / us:>9.3f} {f16 / us:>9.3f}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--ops", default=",".join(OPS))
    ap.add_argument("--json", default=None)
    ap.add_argument("--shapes", default=None,
                    help='N x K list, e.g. "8192x28672,4096x4096" (default: the '
                         "five bench shapes)")
    ap.add_argument("--modes", default="streaming,hot",
                    help="comma-separated subset of " + ",".join(MODES))
    ap.add_argument("--variant", action="append", default=[], metavar="OP=V1,V2",
                    help="variants to time for an op (default: its incumbent)")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the read ceiling (profiling runs)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB, the "
                         "known-size reference of counter (FETCH_SIZE / "
                         "WRITE_SIZE) runs")
    a = ap.parse_args(argv)
    from .. import _capi
    print(f"library: {_capi.version()}", flush=True)   # the build that ran
    ops = tuple(o for o in a.ops.split(",") if o)
    if not ops or any(o not in OPS for o in ops):
        print(f"sweep: --ops must name some of {tuple(OPS)}", file=sys.stderr)
        return 2
    try:
        shapes = (SHAPES if a.shapes is None else
                  [tuple(int(v) for v in s.lower().split("x")) for s in a.shapes.split(",") if s])
        variants = {}
        for spec in a.variant:
            op, vs = spec.split("=", 1)
            variants[op] = [v for v in vs.split(",") if v]
    except ValueError:
        print("sweep: --shapes takes NxK,NxK... and --variant OP=V1,V2", file=sys.stderr)
        return 2
    modes = tuple(m for m in a.modes.split(",") if m)
    if (any(len(sh) != 2 for sh in shapes) or any(m not in MODES for m in modes)
            or any(op not in OPS for op in variants)):
        print("sweep: bad --shapes, --modes or --variant", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("sweep: no GPU visible", file=sys.stderr)
        return 1
    if a.calib_copy_mib:
        src = torch.empty(a.calib_copy_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    recs = run(ops=ops, shapes=shapes, modes=modes, steps=a.steps, warmup=a.warmup,
               variants=variants, ceiling=not a.no_ceiling)
    print(table(recs), flush=True)
    print("\n" + speedups(recs), flush=True)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(recs, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
