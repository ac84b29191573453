"""Per-launch fixed cost and single-launch read bandwidth on this device.

Usage: python -m cudalab_amd.evaluator.floor [--launches 2000] [--json FILE]

Two curves in the bench's window caliber (back-to-back launches on one
stream, queued behind an on-device wait so the host's submission rate is
not what is timed):

  floor    cq_launch_floor: a kernel with no memory work, for every
           (workgroups, threads per workgroup) pair of GRIDS x BLOCKS.
           What one dispatch of that launch shape costs before any kernel
           body runs: command processing, workgroup launch and the
           end-of-kernel release.
  ceiling  cq_read_ceiling: a plain 16-byte-per-thread streaming read of
           BYTES bytes per launch over a rotating pool of distinct buffers
           larger than the 256 MB MALL (HBM-cold), with the fitted line
           t = t0 + bytes / B over the sizes from 8 MB up: t0 is the fixed
           cost per launch of a read and B the bandwidth it streams at.

A GEMV call of b bytes in one launch cannot take less than the ceiling's
time at b bytes: the floor and t0 say how much of a short call is the
launch itself, which no kernel body can remove.
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from .. import _capi
from ..ext import launch_floor, prefill_delay_us, read_ceiling

GRIDS = (1, 64, 128, 256, 512, 1024, 2048, 4096, 8192)
BLOCKS = (64, 256, 512, 1024)
BYTES = (64 << 10, 256 << 10, 1 << 20, 2_172_928, 4 << 20, 8_667_136,
         16 << 20, 23_279_104, 32 << 20, 64 << 20, 128 << 20, 256 << 20)
HBM_PEAK_GBS = 8000.0


def floor_curve(launches: int, warmup: int = 200) -> list[dict]:
    rows = []
    first = True
    for block in BLOCKS:
        for grid in GRIDS:
            us = launch_floor(grid, block, warmup=warmup, n_launches=launches,
                              burn_ms=300.0 if first else 20.0,
                              delay_us=prefill_delay_us(launches))
            first = False
            rows.append({"grid": grid, "block": block, "us_per_launch": round(us, 4)})
    return rows


def ceiling_curve(launches: int, warmup: int = 200) -> list[dict]:
    rows = []
    for b in BYTES:
        # long enough that the window's time, not its edges, dominates
        n = max(200, min(launches, int(4e9 // b)))
        r = read_ceiling(b, warmup=warmup, n_launches=n, burn_ms=100.0,
                         delay_us=prefill_delay_us(n))
        rows.append({"bytes": b, "launches": n, "us_per_launch": round(r["us_per_call"], 4),
                     "GBps": round(r["GBps"], 1),
                     "frac_peak": round(r["GBps"] / HBM_PEAK_GBS, 4)})
        torch.cuda.empty_cache()
    return rows


def fit_line(rows: list[dict], min_bytes: int = 8 << 20) -> dict:
    """Least-squares t = t0 + bytes / B over the sizes >= min_bytes."""
    pts = [(r["bytes"], r["us_per_launch"]) for r in rows if r["bytes"] >= min_bytes]
    n = len(pts)
    mx = sum(p[0] for p in pts) / n
    my = sum(p[1] for p in pts) / n
    sxx = sum((p[0] - mx) ** 2 for p in pts)
    sxy = sum((p[0] - mx) * (p[1] - my) for p in pts)
    slope = sxy / sxx                        # us per byte
    t0 = my - slope * mx
    return {"t0_us": round(t0, 4), "GBps": round(1.0 / slope / 1e3, 1),
            "points": n, "min_bytes": min_bytes}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--launches", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--json", default=None, help="also write the records here")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("floor: no GPU visible", file=sys.stderr)
        return 1
    lib = _capi.load()
    version = lib.cq_version().decode()
    print(f"library: {version}", flush=True)
    fl = floor_curve(a.launches, a.warmup)
    print("launch floor, us per launch (empty kernel; rows: threads per "
          "workgroup, columns: workgroups)", flush=True)
    print("threads " + "".join(f"{g:>9d}" for g in GRIDS))
    for block in BLOCKS:
        vals = [r["us_per_launch"] for r in fl if r["block"] == block]
        print(f"{block:7d} " + "".join(f"{v:9.3f}" for v in vals), flush=True)
    ce = ceiling_curve(a.launches, a.warmup)
    print("read ceiling (one 16-byte load per thread, HBM-cold pool)", flush=True)
    print(f"{'bytes':>12} {'us/launch':>10} {'GB/s':>8} {'of 8 TB/s':>10}")
    for r in ce:
        print(f"{r['bytes']:12d} {r['us_per_launch']:10.3f} {r['GBps']:8.1f} "
              f"{100 * r['frac_peak']:9.1f}%", flush=True)
    fit = fit_line(ce)
    print(f"fit over >= {fit['min_bytes'] >> 20} MiB ({fit['points']} sizes): "
          f"t = {fit['t0_us']:.3f} us + bytes / {fit['GBps']:.0f} GB/s")
    if a.json:
        with open(a.json, "w") as f:
            json.dump({"library": version, "floor": fl, "ceiling": ce, "fit": fit}, f,
                      indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
