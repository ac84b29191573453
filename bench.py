#!/usr/bin/env python
"""Headline benchmark: INT4 W4A16 GEMV 4096x4096, streaming (HBM-cold), on
one MI355X.  Prints ONE JSON line (the driver's contract).

A step is one GEMV call on one set of inputs.  Streaming mode rotates
through a pool of distinct (W_packed, scale, x, y) sets totalling more than
512 MiB, so W is read from HBM on every call (the 256 MB MALL cannot hold
the pool).  The timed loop runs in native code (cq_pool_timing):

  1. untimed launches until both --warmup launches and --burn-ms (300 ms)
     of wall-clock time have passed (the reference's measure_block burns at
     least 300 ms, cudalab/evaluator/bench.py:294-300), then a sync;
  2. a bounded on-device wait (one wave, no memory work) during which the
     host enqueues the whole window, so the window times the GPU and not
     the host's submission rate (about 2.5-3.5 us per launch on MI355X,
     close to the GEMV's own 3.4 us);
  3. the start event, exactly --steps back-to-back launches on one stream,
     the stop event; barrier + torch.cuda.synchronize() around it all.

  value         algorithmic bytes x K / event time of the window (GB/s,
                whole-job throughput, inputs resident in HBM)
  us_per_call   event time of the window / K
  rocprof_isolated_dispatch_us
                the committed rocprofv3 kernel-trace average of the same
                kernel instance and shape (profiles/, read at run time), when
                the profile matches the plan that ran: an isolated-dispatch
                caliber (the profiler serialises every dispatch behind a
                completion signal), not the kernel's time per call
  roofline      algorithmic bytes / us_per_call against 8 TB/s.  `traffic`
                is the measured HBM bytes per launch from the committed
                rocprofv3 counter summary.  `measured_ceiling` is a plain read
                of the same bytes per launch (cq_read_ceiling) over an equally
                cold pool in the same window caliber: what one launch of this
                size can reach.  `launch_floor_us` is an empty kernel of the
                GEMV's grid and workgroup size, same caliber.  `kernel_body`
                is the on-device span of one launch (first wave start to last
                y store, from the wave timeline); `isolated_dispatch` holds
                the rocprof figure above as bytes / duration.
  detail        the same window (K launches, pre-filled) repeated: INT4
                streaming, INT4 hot (one resident set), INT8 streaming on the
                same shape, each the median of 5 windows, and their ratios;
                plus the hipGraph and grouped (8 GEMVs per launch) calibers,
                and one window timed as the host issues it (no wait ahead:
                the reference's method).  A window whose enqueue outlasted
                its wait is timed again behind a longer one, and says so.
  cpu_baseline  the oracle's fused OpenMP CPU GEMV (oracle/qgemv_oracle.c)
                on the same shape, timed on this host over a bounded sample:
                about --cpu-seconds (6 s) of calls cycling over 16 distinct
                host-resident sets of the pool, median per call; beside it
                the same C port on one thread, the reference's torch CPU
                formulation (dequantize, FP32 torch.mv) on all threads and
                on one, and the host CPU model (about 13 s of CPU in all)

`--cpu-sweep` instead times the CPU paths alone at the five bench shapes
(INT4 and INT8; C port and torch formulation; all threads and one) and
prints one JSON line per shape (no GPU needed).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
BASELINE = json.loads((ROOT / "BASELINE.json").read_text())
METRIC = BASELINE["metric"]
HBM_PEAK_GBS = 8000.0
# launches per window of the secondary figures in `detail` (INT4 windows,
# hot, INT8, read ceiling, launch floor), at least --steps
DETAIL_LAUNCHES = 2000
TRAFFIC_FILE = ROOT / "profiles" / "int4gemv_4096x4096_streaming_traffic.json"


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--burn-ms", type=float, default=300.0,
                    help="untimed launches run for at least this long before "
                         "the window (as well as --warmup launches)")
    ap.add_argument("--variant", default="int4gemv_cdna4")
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--k", type=int, default=4096)
    ap.add_argument("--mode", choices=("streaming", "hot"), default="streaming")
    ap.add_argument("--cpu-seconds", type=float, default=6.0,
                    help="CPU baseline sample: seconds of the all-thread C port "
                         "(half that on one thread, a third per thread count for "
                         "the torch formulation)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--no-detail", action="store_true",
                    help="skip the INT8 / hot-mode / ceiling detail measurements")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB "
                         "(counter calibration runs)")
    ap.add_argument("--cpu-sweep", action="store_true",
                    help="time only the CPU paths at the five bench shapes")
    ap.add_argument("--prefill-us", type=float, default=None,
                    help="on-device wait queued before the headline window "
                         "(default: 5 us per launch + 0.5 ms); profiling runs, "
                         "whose host submission is slower, need more")
    return ap.parse_args(argv)


def gpu_loop(op: str, variant: str, sets, steps: int, warmup: int,
             burn_ms: float, delay_us: float | None = None) -> dict:
    """One window of `steps` back-to-back launches rotating through `sets`,
    pre-filled behind an on-device wait, timed by two HIP events around the
    window (native loop, no per-launch events)."""
    import torch
    from cudalab_amd.ext import pool_timing, prefill_delay_us
    d = prefill_delay_us(steps) if delay_us is None else delay_us
    torch.cuda.synchronize()           # barrier (single rank) + sync
    t0 = time.perf_counter()
    r = pool_timing(op, variant, sets, warmup=warmup, n_launches=steps,
                    per_kernel=False, burn_ms=burn_ms, delay_us=d)
    retried = False
    if d > 0 and not r["prefilled"]:
        # the host took longer to enqueue the window than the wait lasted,
        # so the GPU may have idled inside it: time it again with a wait
        # twice the enqueue time (no new burn: the clocks are settled)
        retried = True
        d = min(1e6, 2.0 * r["host_us"] + 500.0)
        r = pool_timing(op, variant, sets, warmup=warmup, n_launches=steps,
                        per_kernel=False, delay_us=d)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    return {"total_us": r["total_us"], "us_per_call": r["total_us"] / steps,
            "host_us_per_call": r["host_us"] / steps, "wall_s": wall_s,
            "delay_us": d, "prefilled": r["prefilled"], "retried": retried}


def windows(op: str, variant: str, sets, steps: int, count: int = 5) -> dict:
    """`count` more pre-filled windows of `steps` launches (no burn: the
    caller has just run one); median and spread of µs per call.  The pool
    rotation continues from window to window (each call of the native loop
    starts at its list's first set), so a short window never meets sets
    that the previous one left in the MALL."""
    from cudalab_amd.ext import pool_timing, prefill_delay_us
    us = []
    off = 0
    uncovered = 0
    for _ in range(count):
        rot = sets[off:] + sets[:off]
        d = prefill_delay_us(steps)
        r = pool_timing(op, variant, rot, warmup=0, n_launches=steps,
                        per_kernel=False, delay_us=d)
        if not r["prefilled"]:     # enqueue outlasted the wait: time it again
            uncovered += 1
            r = pool_timing(op, variant, rot, warmup=0, n_launches=steps,
                            per_kernel=False,
                            delay_us=min(1e6, 2.0 * r["host_us"] + 500.0))
        off = (off + steps) % len(sets)
        us.append(r["total_us"] / steps)
    us.sort()
    return {"median": us[len(us) // 2], "min": us[0], "max": us[-1], "n": count,
            "rerun_uncovered": uncovered}


def unfilled_window(op: str, variant: str, sets, steps: int) -> dict:
    """One window with no on-device wait ahead of it: the launches are timed
    as the host issues them, the way the reference's measure_block times a
    block between two events (cudalab/evaluator/bench.py:294-309).  Kept
    beside the pre-filled figure so the two methods stay comparable."""
    from cudalab_amd.ext import pool_timing
    r = pool_timing(op, variant, sets, warmup=0, n_launches=steps,
                    per_kernel=False, delay_us=0.0)
    return {"us_per_call": r["total_us"] / steps,
            "host_us_per_call": r["host_us"] / steps}


def kernel_instance(plan: dict) -> str:
    """Name fragment of the kernel instance a plan launches (as rocprofv3
    prints it), e.g. 'int4gemv_lds_kernel<64, 2, 1, 512>'."""
    if plan["kernel"] == "lds":
        return (f"int4gemv_lds_kernel<{plan['cw']}, {plan['j']}, {plan['r']}, "
                f"{plan['block']}>")
    if plan["kernel"] == "tiled":
        return f"int4gemv_tiled_kernel<256, {plan['tile']}, {plan['r']}>"
    return f"int4gemv_{plan['kernel']}"


def load_rocprof(N: int, K: int, mode: str, plan: dict):
    """The committed kernel-trace record for this shape, if it is of the
    kernel instance that ran: (mean µs per dispatch, file name) or
    (None, reason)."""
    f = ROOT / "profiles" / f"int4gemv_{N}x{K}_{mode}_kernel_trace.json"
    if not f.exists():
        return None, f"no {f.name}"
    try:
        d = json.loads(f.read_text())
    except Exception as e:  # noqa: BLE001
        return None, f"{f.name}: {e}"
    want = kernel_instance(plan)
    if want not in d.get("kernel", "") or d.get("shape") != [N, K]:
        return None, (f"{f.name} is of {d.get('kernel', '?')[:60]} "
                      f"{d.get('shape')}, not {want} [{N}, {K}]")
    return round(float(d["mean_us"]), 4), f"profiles/{f.name}"


def make_sets(op: str, N: int, K: int, mode: str, seed: int = 1234):
    from cudalab_amd.evaluator.sweep import make_sets as _make_sets
    return _make_sets(op, N, K, mode, seed)


def graph_loop(ext, variant: str, sets, per_graph: int = 256,
               replays: int = 20) -> float:
    """Per-call time of `per_graph` launches captured in one HIP graph,
    replayed `replays` times (launch-overhead-amortized caliber)."""
    import torch
    for (W, s, x, o) in sets[:4]:
        ext.forward_into(variant, W, s, x, o)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=side):
        for i in range(per_graph):
            W, s, x, o = sets[i % len(sets)]
            ext.forward_into(variant, W, s, x, o)
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (per_graph * replays)


def grouped_graph_loop(ext, variant: str, sets, group: int = 8,
                       per_graph: int = 32, replays: int = 20) -> float:
    """Per-problem time of grouped launches (`group` independent problems
    of the pool in one launch, cq_int4gemv_grouped), `per_graph` of them
    captured in one HIP graph over distinct sets, replayed `replays` times:
    the kernel's bandwidth with the per-launch floor shared by `group`
    GEMVs."""
    import torch
    n = len(sets) // group * group
    groups = [sets[i:i + group] for i in range(0, n, group)]
    ext.forward_grouped(variant, groups[0])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=side):
        for i in range(per_graph):
            ext.forward_grouped(variant, groups[i % len(groups)])
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (per_graph * replays * group)


def _timed_calls(fn, min_s: float, min_n: int, max_n: int) -> list[float]:
    """Seconds of each call fn(i), i = 0, 1, ..., until at least `min_s`
    seconds and `min_n` calls have run (at most `max_n` calls)."""
    ts: list[float] = []
    t_end = time.perf_counter() + min_s
    while len(ts) < max_n and (len(ts) < min_n or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn(len(ts))
        ts.append(time.perf_counter() - t0)
    return ts


def cpu_baseline(N: int, K: int, sets, seconds: float = 6.0,
                 max_sets: int = 16) -> dict:
    """The oracle's fused C + OpenMP GEMV, timed on this host over a bounded
    sample of the bench workload: the first `max_sets` sets of the pool,
    copied to host memory (untimed), cycled call by call for about
    `seconds` with all threads, then about seconds/2 on one thread.  Beside
    it the reference's torch CPU formulation, about seconds/3 per thread
    count.  Medians per call."""
    from oracle import oracle as orc
    from cudalab_amd.operators.int4gemv import int4_bytes
    host = [(wp.cpu().numpy(), s.cpu().numpy(), x.cpu().numpy())
            for (wp, s, x, _) in sets[:max_sets]]
    m = len(host)
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or min(16, os.cpu_count() or 1)
    wpn, sn, xn = host[0]
    y = orc.gemv_w4_cpu(wpn, sn, xn, threads)
    ex, S = orc.exact_w4(wpn, sn, xn)
    assert orc.arith_ratio(y, ex, S, K).max() <= 1.0
    for i in range(3):
        orc.gemv_w4_cpu(*host[i % m], threads)
    many = _timed_calls(lambda i: orc.gemv_w4_cpu(*host[i % m], threads),
                        seconds, 20, 200000)
    one = _timed_calls(lambda i: orc.gemv_w4_cpu(*host[i % m], 1),
                       seconds / 2, 5, 100000)
    torch_all, torch_one, torch_n = _torch_cpu_us(sets[:max_sets], threads, seconds / 3)
    med = statistics.median(many)
    bytes_ = int4_bytes(N, K)
    total_s = sum(many) + sum(one)
    return {"value": round(bytes_ / med / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"{len(many)} calls of the INT4 {N}x{K} GEMV ({sum(many):.1f} s "
                      f"of CPU work on {threads} threads), cycling over {m} distinct "
                      f"host-resident input sets of the bench pool "
                      f"({m * bytes_ / 1e6:.0f} MB), after 3 warm-up calls; median "
                      f"{med * 1e6:.1f} us per call; fused unpack-dequant-dot in "
                      f"C + OpenMP (oracle/qgemv_oracle.c)",
            "us_per_call": round(med * 1e6, 2),
            "c_port_1_thread_us": round(statistics.median(one) * 1e6, 1),
            "c_port_1_thread_calls": len(one),
            "sample_cpu_seconds": round(total_s, 2),
            "torch_formulation_us": {"threads": threads, "all_threads": round(torch_all, 1),
                                     "one_thread": round(torch_one, 1),
                                     "calls": torch_n,
                                     "what": "dequantize_w(W_packed, scale) then "
                                             "torch.mv(Wd, x.float()).half() on the CPU "
                                             "(cudalab/int4gemv_correctness.py:220-221), "
                                             "cycling over the same sets, median per call "
                                             "after 1 warm-up call"},
            "host": _host_cpu()}


def _torch_cpu_us(sets, threads: int, seconds: float) -> tuple[float, float, list[int]]:
    """The reference's CPU path (dequantize then an FP32 torch.mv) over
    host copies of `sets`, with `threads` threads and with one: median us
    per call and the call counts."""
    import torch
    from cudalab_amd.int4gemv_quantize import dequantize_w
    host = [(wp.cpu(), s.cpu(), x.cpu()) for (wp, s, x, _) in sets]

    def call(i):
        wp, s, x = host[i % len(host)]
        torch.mv(dequantize_w(wp, s), x.float()).half()
    prev = torch.get_num_threads()
    out = []
    try:
        for t in (threads, 1):
            torch.set_num_threads(t)
            call(0)
            out.append(_timed_calls(call, seconds, 3, 10000))
    finally:
        torch.set_num_threads(prev)
    return (statistics.median(out[0]) * 1e6, statistics.median(out[1]) * 1e6,
            [len(out[0]), len(out[1])])


def _host_cpu() -> dict:
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count()}


def load_traffic(N: int, K: int):
    if not TRAFFIC_FILE.exists():
        return None
    try:
        d = json.loads(TRAFFIC_FILE.read_text())
        if d.get("shape") == [N, K]:
            return d.get("hbm_bytes_per_launch")
    except Exception:  # noqa: BLE001
        return None
    return None


CPU_SWEEP_SHAPES = ((1024, 4096), (4096, 1024), (4096, 4096), (11008, 4096),
                    (4096, 11008))


def cpu_sweep(seconds: float = 1.0) -> int:
    """The CPU paths at the five bench shapes, INT4 and INT8: the oracle's
    fused C + OpenMP port on all threads and on one, and the reference's
    torch CPU formulation (INT4: dequantize_w then an FP32 torch.mv,
    cudalab/int4gemv_correctness.py:220-221; INT8: W_q.float() * scale then
    torch.mv, cudalab/qgemv_correctness.py:189) on all threads and on one.
    Each figure is the median per call of about `seconds` of calls (at least
    3) on one input set drawn with the bench recipe (W ~ N(0, 0.02)
    quantized, x ~ N(0, 1)); each result is checked against the oracle's
    bound first.  One JSON line per (op, shape)."""
    import torch
    from oracle import oracle as orc
    from cudalab_amd.int4gemv_quantize import dequantize_w
    from cudalab_amd.operators import int4gemv as op4
    from cudalab_amd.operators import qgemv as op8
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or min(16, os.cpu_count() or 1)
    host = _host_cpu()

    def med_us(fn, n_min=3):
        fn()
        return statistics.median(_timed_calls(lambda i: fn(), seconds, n_min, 100000)) * 1e6

    prev = torch.get_num_threads()
    try:
        for op in ("int4gemv", "qgemv"):
            for (N, K) in CPU_SWEEP_SHAPES:
                if op == "int4gemv":
                    wp, sc, x, _ = op4.device_random_set(N, K, 1234 + 100000, device="cpu")
                    a = (wp.numpy(), sc.numpy(), x.numpy())
                    y = orc.gemv_w4_cpu(*a, threads)
                    assert orc.check_w4(y, *a) <= 1.0
                    c_fn = orc.gemv_w4_cpu
                    nbytes = op4.int4_bytes(N, K)

                    def t_fn(wp=wp, sc=sc, x=x):
                        torch.mv(dequantize_w(wp, sc), x.float()).half()
                else:
                    wq, sc, x, _ = op8.device_random_set(N, K, 1234 + 100000, device="cpu")
                    a = (wq.numpy(), sc.numpy(), x.numpy())
                    y = orc.gemv_w8_cpu(*a, threads)
                    assert orc.check_w8(y, *a) <= 1.0
                    c_fn = orc.gemv_w8_cpu
                    nbytes = op8.q8_bytes(N, K)

                    def t_fn(wq=wq, sc=sc, x=x):
                        torch.mv(wq.float() * sc[:, None], x.float()).half()
                rec = {"op": op, "N": N, "K": K, "algorithmic_bytes": nbytes,
                       "threads": threads}
                rec["c_port_us"] = round(med_us(lambda: c_fn(*a, threads)), 2)
                rec["c_port_1_thread_us"] = round(med_us(lambda: c_fn(*a, 1)), 2)
                torch.set_num_threads(threads)
                rec["torch_us"] = round(med_us(t_fn), 1)
                torch.set_num_threads(1)
                rec["torch_1_thread_us"] = round(med_us(t_fn), 1)
                torch.set_num_threads(prev)
                rec["c_port_GBps"] = round(nbytes / rec["c_port_us"] / 1e3, 2)
                rec["host"] = host
                print(json.dumps(rec), flush=True)
    finally:
        torch.set_num_threads(prev)
    return 0


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is "
              "not supported (each GPU would run the same kernel on its own "
              "row shard of W; only the one-GPU figure is measured)",
              file=sys.stderr)
        return 2
    if args.cpu_sweep:
        return cpu_sweep()
    import torch
    from cudalab_amd.build import build
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    ext4 = build("int4gemv")
    N, K = args.n, args.k
    sets, nbytes = make_sets("int4gemv", N, K, args.mode)
    for (wp, s, x, out) in sets[:1]:
        ext4.forward_into(args.variant, wp, s, x, out)   # validate once
    plan = ext4.describe(args.variant, sets[0][0], sets[0][2])

    if args.calib_copy_mib:
        src = torch.empty(args.calib_copy_mib << 20, dtype=torch.uint8,
                          device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()

    r = gpu_loop("int4gemv", args.variant, sets, args.steps, args.warmup,
                 args.burn_ms, args.prefill_us)

    total_s = r["total_us"] * 1e-6
    value = nbytes * args.steps / total_s / 1e9
    achieved = nbytes / (r["us_per_call"] * 1e-6) / 1e9
    traffic = load_traffic(N, K)
    rp_us, rp_src = load_rocprof(N, K, args.mode, plan)

    from cudalab_amd import _capi
    detail = {"library": _capi.load().cq_version().decode(),
              "plan": plan, "kernel_instance": kernel_instance(plan),
              "pool_sets": len(sets), "pool_bytes": len(sets) * nbytes,
              "algorithmic_bytes_per_call": nbytes,
              "window": {"launches": args.steps, "warmup_launches_min": args.warmup,
                         "burn_ms_min": args.burn_ms,
                         "prefill": "on-device wait queued before the start "
                                    "event; the host enqueues the window behind it",
                         "host_enqueue_us_per_call": round(r["host_us_per_call"], 4),
                         "wait_us": round(r["delay_us"], 1),
                         "wait_covered_enqueue": r["prefilled"],
                         "rerun_after_uncovered_wait": r["retried"]},
              "wall_s_timed": round(r["wall_s"], 4),
              "rocprof_source": rp_src}
    ceil = floor_us = body_span_us = None
    if not args.no_detail:
        from cudalab_amd.ext import launch_floor, prefill_delay_us, read_ceiling
        # every secondary window has one fixed length whatever --steps says,
        # so INT4, INT8, hot, the ceiling and the floor compare like for like
        nl = max(args.steps, DETAIL_LAUNCHES)
        ceil = read_ceiling(nbytes, warmup=args.warmup, n_launches=nl,
                            burn_ms=100.0, delay_us=prefill_delay_us(nl))
        floor_us = launch_floor(int(plan["grid"]), int(plan["block"]),
                                warmup=args.warmup, n_launches=nl, burn_ms=100.0,
                                delay_us=prefill_delay_us(nl))
        w4 = windows("int4gemv", args.variant, sets, nl)
        detail["int4_5_windows_us"] = {k: round(v, 4) for k, v in w4.items()}
        uw = unfilled_window("int4gemv", args.variant, sets, nl)
        detail["int4_unfilled_window"] = {
            "us_per_call": round(uw["us_per_call"], 4),
            "host_enqueue_us_per_call": round(uw["host_us_per_call"], 4),
            "note": f"{nl} launches timed as the host issues them (no on-device "
                    "wait ahead of the window: the reference's measure_block "
                    "method and this bench's method before the pre-filled window); "
                    "bound by the slower of the host's enqueue and the GPU"}
        detail["graph_us_per_call"] = round(graph_loop(ext4, args.variant, sets), 4)
        if args.mode == "streaming" and len(sets) >= 16:
            gp = grouped_graph_loop(ext4, args.variant, sets)
            detail["grouped8_graph_us_per_gemv"] = round(gp, 4)
            detail["grouped8_graph_GBps"] = round(nbytes / gp / 1e3, 1)
            detail["grouped8_note"] = ("8 independent GEMVs of this shape per launch "
                                       "(cq_int4gemv_grouped) over distinct HBM-cold "
                                       "sets, from a HIP graph: the per-launch cost "
                                       "shared by 8 GEMVs; not the headline caliber")
        if plan.get("kernel") == "lds":
            from cudalab_amd.evaluator.timeline import by_workgroup, run_stamped, summarize
            tl = run_stamped(args.variant, sets, n_launches=400, warmup=args.warmup,
                             burn_ms=100.0)
            ts = summarize(tl["stamps"], tl["ticks_per_us"])
            bw = by_workgroup(tl["stamps"], tl["ticks_per_us"], int(plan["block"]) // 64)
            body_span_us = ts["span_us"]
            detail["wave_timeline"] = {
                "span_us": round(ts["span_us"], 3),
                "gap_us": round(ts["gap_us"], 3),
                "points_us": {p: [round(v["p50_us"], 3), round(v["max_us"], 3)]
                              for p, v in ts["points"].items()},
                "instrumented_us_per_call": round(tl["us_per_launch"], 4),
                "x_barrier_by_workgroup_us": {
                    "first_on_cu": round(bw["barrier_first_on_cu_us"], 3),
                    "second_on_cu": (round(bw["barrier_second_on_cu_us"], 3)
                                     if bw["barrier_second_on_cu_us"] is not None else None),
                    "per_xcd": [round(v, 3) for v in bw["barrier_by_xcd_us"]],
                    "corr_start_barrier": round(bw["corr_start_barrier"], 3)},
                "note": "cq_int4_timeline over the same pool: a stamped copy of this "
                        "plan's kernel (same arithmetic and launch shape), 400 "
                        "launches; per point [median wave, last wave] in us from "
                        "each launch's first wave start; span = first wave start "
                        "to last y store, gap = last y store to the next launch's "
                        "first wave start (medians over launches); the x barrier per "
                        "workgroup: the workgroup that started first on its CU and "
                        "the second, per XCD, and its correlation with the "
                        "workgroup's start"}
        gpu_loop("int4gemv", args.variant, sets[:1], nl, args.warmup, 100.0)
        h = windows("int4gemv", args.variant, sets[:1], nl)
        detail["hot_us_per_call"] = round(h["median"], 4)
        detail["hot_GBps"] = round(nbytes / h["median"] / 1e3, 1)
        build("qgemv")
        q_sets, q_bytes = make_sets("qgemv", N, K, args.mode)
        gpu_loop("qgemv", "qgemv_cdna4", q_sets, nl, args.warmup, 100.0)
        q = windows("qgemv", "qgemv_cdna4", q_sets, nl)
        detail["int8_us_per_call"] = round(q["median"], 4)
        detail["int8_GBps"] = round(q_bytes / q["median"] / 1e3, 1)
        detail["speedup_int4_vs_int8"] = round(q["median"] / w4["median"], 3)
        detail["speedup_note"] = ("INT8 and INT4 medians of 5 pre-filled windows of "
                                  f"{nl} launches each, streaming, same shape")
        del q_sets
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(N, K, sets, seconds=args.cpu_seconds)

    roofline = {"bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic}
    if body_span_us is not None:
        roofline["kernel_body"] = {
            "span_us": round(body_span_us, 3),
            "GBps": round(nbytes / body_span_us / 1e3, 1),
            "frac": round(nbytes / body_span_us / 1e3 / HBM_PEAK_GBS, 4),
            "note": "on-device figure: first wave start to last y store of one "
                    "launch (wave timeline, median over launches); the call's "
                    "other time is the gap to the next launch's first wave"}
    if rp_us is not None:
        roofline["isolated_dispatch"] = {
            "us": rp_us,
            "achieved": round(nbytes / rp_us / 1e3, 1),
            "frac": round(nbytes / rp_us / 1e3 / HBM_PEAK_GBS, 4),
            "note": "rocprofv3 --kernel-trace caliber: each dispatch is "
                    "serialised behind a completion signal and starts on an "
                    "idle GPU; a different caliber from the back-to-back "
                    "window, not this kernel's time per call"}
    if ceil is not None:
        roofline.update({
            "measured_ceiling": round(ceil["GBps"], 1),
            "frac_of_measured_ceiling": round(achieved / ceil["GBps"], 4),
            "ceiling_note": "plain streaming read of the same bytes per launch "
                            "over an HBM-cold pool (cq_read_ceiling), same "
                            "pre-filled window caliber",
            "launch_floor_us": round(floor_us, 4),
            "floor_note": "back-to-back launches of a kernel with no memory work "
                          "in the GEMV's launch shape (cq_launch_floor, grid %s x "
                          "%s threads), same caliber" % (plan["grid"], plan["block"])})
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_s * 1e3 / args.steps, 6),
        "us_per_call": round(r["us_per_call"], 4),
        "rocprof_isolated_dispatch_us": rp_us,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic: W ~ N(0,0.02) fp16 quantized G=128, x ~ N(0,1) "
                "fp16, drawn on the device",
        "config": {"workload": f"INT4 W4A16 GEMV {N}x{K} {args.mode} "
                               f"({'HBM-cold pool of %d distinct sets' % detail['pool_sets'] if args.mode == 'streaming' else 'single resident set'})",
                   "N": N, "K": K, "group_size": 128,
                   "variant": args.variant, "mode": args.mode,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
