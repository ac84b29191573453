"""Wave timeline of the INT4 GEMV: where the time of one call goes.

Usage: python -m cudalab_amd.evaluator.timeline [--n 4096] [--k 4096]
       [--variant int4gemv_cdna4] [--launches 400] [--json FILE]

Runs the bench's streaming workload (an HBM-cold pool of distinct sets) in
the bench's window caliber through cq_int4_timeline: a copy of the LDS
kernel the variant plans for (n, k), with the same arithmetic, launch shape
and outputs, whose waves stamp the 100 MHz wall clock at five points: wave
start, after the x barrier, after the first and the last weight chunk are
summed, after the y stores are issued.  Per launch, times are taken from
the launch's first wave start; the report gives the median over launches
of each point's median and maximum over the waves, the span (first wave
start to last store), the gap from a launch's last store to the next
launch's first wave start, and the x barrier per workgroup: of the
workgroup that started first on its CU and of the second, per XCD, and
its correlation with the workgroup's start (by_workgroup).  The same pool
is timed through the product kernel (cq_pool_timing) beside it: the stamps
cost a little (their stores and clock reads), so the instrumented rate is a
little slower.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import sys

import numpy as np
import torch

from .. import _capi

POINTS = ("wave start", "x barrier", "first chunk summed",
          "last chunk summed", "y stored")


def run_stamped(variant: str, sets: list, n_launches: int, warmup: int = 200,
                burn_ms: float = 300.0, delay_us: float | None = None) -> dict:
    """cq_int4_timeline over `sets` ((W, scale, x, out) tuples of one shape).
    Returns {"stamps": int64 array (n_launches, waves, 8) in launch order,
    "ticks_per_us", "waves", "us_per_launch"}."""
    from ..ext import Int4gemvExt, prefill_delay_us
    lib = _capi.load()
    W0, _, x0, _ = sets[0]
    N, K = W0.size(0), 2 * W0.size(1)
    d = Int4gemvExt().describe(variant, W0, x0)
    if d.get("kernel") != "lds":
        raise RuntimeError(f"the timeline covers the LDS kernel; {variant} plans "
                           f"{d.get('kernel')} for {N}x{K}")
    waves = int(d["grid"]) * int(d["block"]) // 64
    stamps = torch.zeros(n_launches * waves * 8, dtype=torch.int64, device=W0.device)
    n = len(sets)
    VP = ctypes.c_void_p * n
    w = VP(*[s[0].data_ptr() for s in sets])
    sc = VP(*[s[1].data_ptr() for s in sets])
    xs = VP(*[s[2].data_ptr() for s in sets])
    ys = VP(*[s[3].data_ptr() for s in sets])
    waves_out = ctypes.c_int64(0)
    tpu = ctypes.c_double(0.0)
    tot = ctypes.c_double(0.0)
    if delay_us is None:
        delay_us = prefill_delay_us(n_launches)
    with torch.cuda.device(W0.device):
        s = torch.cuda.current_stream(W0.device)
        torch.cuda.synchronize()
        st = lib.cq_int4_timeline(variant.encode(), w, sc, xs, ys, n, N, K,
                                  s.cuda_stream, warmup, float(burn_ms),
                                  float(delay_us), n_launches, stamps.data_ptr(),
                                  stamps.numel(), ctypes.byref(waves_out),
                                  ctypes.byref(tpu), ctypes.byref(tot))
        torch.cuda.synchronize()
    if st != _capi.CQ_OK:
        raise RuntimeError(f"cq_int4_timeline failed (status {st}): {_capi.last_error()}")
    if waves_out.value != waves:
        raise RuntimeError(f"waves per launch {waves_out.value}, expected {waves}")
    a = stamps.cpu().numpy().reshape(n_launches, waves, 8)
    order = np.argsort(a[:, :, 0].min(axis=1), kind="stable")
    return {"stamps": a[order], "ticks_per_us": tpu.value, "waves": waves,
            "us_per_launch": tot.value / n_launches}


def summarize(stamps: np.ndarray, ticks_per_us: float, skip: float = 0.25) -> dict:
    """Reduce stamps (launches, waves, 8) to the report's figures, in µs.
    The first `skip` fraction of launches is left out (the window's first
    launches start on an idle GPU), and the last launch has no successor
    for the gap."""
    L = stamps.shape[0]
    lo = min(int(L * skip), max(0, L - 2))
    per = {p: {"p50": [], "max": []} for p in POINTS}
    span, gap = [], []
    for i in range(lo, L - 1):
        t = stamps[i, :, :5].astype(np.float64)
        t0 = t[:, 0].min()
        rel = (t - t0) / ticks_per_us
        for j, p in enumerate(POINTS):
            per[p]["p50"].append(float(np.median(rel[:, j])))
            per[p]["max"].append(float(rel[:, j].max()))
        end = t[:, 4].max()
        span.append(float((end - t0) / ticks_per_us))
        nxt = stamps[i + 1, :, 0].astype(np.float64).min()
        gap.append(float((nxt - end) / ticks_per_us))
    med = statistics.median
    out = {p: {"p50_us": med(v["p50"]), "max_us": med(v["max"])} for p, v in per.items()}
    return {"points": out, "span_us": med(span), "gap_us": med(gap),
            "launches_used": len(span)}


def xcd_of_logical_block(grid: int) -> np.ndarray:
    """XCD of each logical block under the kernels' XCD-contiguous mapping:
    workgroup i runs on XCD i % 8 and each XCD owns one contiguous range of
    logical blocks (cq_kernels.hip, xcd_contiguous_block)."""
    q, r = divmod(grid, 8)
    starts = [x * q + min(x, r) for x in range(9)]
    out = np.empty(grid, dtype=np.int64)
    for x in range(8):
        out[starts[x]:starts[x + 1]] = x
    return out


def by_workgroup(stamps: np.ndarray, ticks_per_us: float, waves_per_group: int,
                 skip: float = 0.25) -> dict:
    """Per-workgroup view of the stamps (launches, waves, 8), waves in
    logical-block order.  A workgroup's barrier time is its waves' latest
    x-barrier stamp (they all wait at one barrier), its start their earliest
    start, both from the launch's first wave start.  Workgroups of one launch
    that share a CU (their XCD and hardware CU id, stamp word 5) are ranked
    by start: the report gives the median barrier of the workgroup that
    started first on its CU and of the second, each XCD's median, and the
    correlation of a workgroup's start with its barrier."""
    L, W, _ = stamps.shape
    if W % waves_per_group:
        raise ValueError("waves per launch not a multiple of the workgroup's waves")
    grid = W // waves_per_group
    lo = min(int(L * skip), max(0, L - 1))
    t = stamps[lo:, :, :5].astype(np.float64)
    rel = (t - t[:, :, 0].min(axis=1)[:, None, None]) / ticks_per_us
    start = rel[:, :, 0].reshape(-1, grid, waves_per_group).min(axis=2)
    barrier = rel[:, :, 1].reshape(-1, grid, waves_per_group).max(axis=2)
    xcd = xcd_of_logical_block(grid)
    # a CU is keyed by its XCD and its hardware CU id (the id alone need not
    # distinguish XCDs)
    cu = (stamps[lo:, :, 5].reshape(-1, grid, waves_per_group)[:, :, 0].astype(np.int64)
          + (xcd.astype(np.int64) << 32)[None, :])
    first, second = [], []
    for i in range(start.shape[0]):
        order = np.lexsort((start[i], cu[i]))
        rank = np.zeros(grid, dtype=np.int64)
        for a, b in zip(order[:-1], order[1:]):
            if cu[i][b] == cu[i][a]:
                rank[b] = rank[a] + 1
        first.append(float(np.median(barrier[i][rank == 0])))
        if (rank == 1).any():
            second.append(float(np.median(barrier[i][rank == 1])))
    per_xcd = [float(np.median(np.median(barrier[:, xcd == x], axis=1)))
               for x in range(8) if (xcd == x).any()]
    return {"workgroups": grid, "launches_used": int(start.shape[0]),
            "barrier_first_on_cu_us": statistics.median(first),
            "barrier_second_on_cu_us": statistics.median(second) if second else None,
            "barrier_by_xcd_us": per_xcd,
            "corr_start_barrier": _corr(start.ravel(), barrier.ravel())}


def _corr(a: np.ndarray, b: np.ndarray) -> float:
    """Pearson correlation, NaN when either side is constant."""
    if a.std() == 0 or b.std() == 0:
        return float("nan")
    return float(np.corrcoef(a, b)[0, 1])


def run(n: int = 4096, k: int = 4096, variant: str = "int4gemv_cdna4",
        n_launches: int = 400) -> dict:
    from .sweep import make_sets, window_us
    sets, nbytes = make_sets("int4gemv", n, k, "streaming")
    r = run_stamped(variant, sets, n_launches)
    s = summarize(r["stamps"], r["ticks_per_us"])
    W0, _, x0, _ = sets[0]
    from ..ext import Int4gemvExt
    wpg = int(Int4gemvExt().describe(variant, W0, x0)["block"]) // 64
    s["by_workgroup"] = by_workgroup(r["stamps"], r["ticks_per_us"], wpg)
    product = window_us("int4gemv", variant, sets, steps=2000, warmup=200)
    return {"variant": variant, "N": n, "K": k, "pool_sets": len(sets),
            "algorithmic_bytes": nbytes, "waves_per_launch": r["waves"],
            "launches": n_launches, "instrumented_us_per_call": r["us_per_launch"],
            "product_us_per_call": product, **s}


def table(rec: dict) -> str:
    lines = [f"INT4 {rec['N']}x{rec['K']} streaming ({rec['pool_sets']} sets), "
             f"{rec['waves_per_launch']} waves per launch, {rec['launches']} stamped "
             f"launches ({rec['launches_used']} used)",
             f"instrumented {rec['instrumented_us_per_call']:.3f} us per call; "
             f"product kernel on the same pool {rec['product_us_per_call']:.3f} us",
             "us from the launch's first wave start (median over launches):",
             f"  {'point':<22} {'median wave':>12} {'last wave':>10}"]
    for p in POINTS:
        v = rec["points"][p]
        lines.append(f"  {p:<22} {v['p50_us']:>12.2f} {v['max_us']:>10.2f}")
    lines.append(f"  span, first wave start .. last y store: {rec['span_us']:.2f}")
    lines.append(f"  gap, last y store .. next launch's first wave start: {rec['gap_us']:.2f}")
    g = rec.get("by_workgroup")
    if g:
        sec = g["barrier_second_on_cu_us"]
        lines.append(f"  x barrier by workgroup ({g['workgroups']} per launch): first to start "
                     f"on its CU {g['barrier_first_on_cu_us']:.2f}, second "
                     + (f"{sec:.2f}" if sec is not None else "-")
                     + f"; per XCD " + " ".join(f"{v:.2f}" for v in g["barrier_by_xcd_us"])
                     + f"; corr(start, barrier) {g['corr_start_barrier']:.2f}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--k", type=int, default=4096)
    ap.add_argument("--variant", default="int4gemv_cdna4")
    ap.add_argument("--launches", type=int, default=400)
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    print(f"library: {_capi.version()}", flush=True)   # the build that ran
    if args.launches < 2 or args.n < 1 or args.k < 128 or args.k % 128:
        print("timeline: --launches >= 2, --n >= 1 and --k a positive multiple of 128",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("timeline: no GPU visible", file=sys.stderr)
        return 1
    rec = run(args.n, args.k, args.variant, args.launches)
    print(table(rec), flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(rec, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
