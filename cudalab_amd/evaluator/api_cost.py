"""Host time per call of the eager API paths.

Usage: python -m cudalab_amd.evaluator.api_cost [--n 4096] [--k 4096]
       [--calls 1000] [--reps 7] [--json FILE]

Each path is called `calls` times back to back right after a long on-device
wait (torch.cuda._sleep) has been enqueued on the same stream, so every call
is enqueued while the GPU is still busy with the wait: the host loop is
never throttled by a full queue and the time is the host's alone.  A sample
counts only if the wait was still running when the loop ended (checked with
an event recorded after it; a loop that outran its wait is discarded and the
wait doubled); the median over `reps` samples is reported.

First the floor: the library's own C loop enqueueing the same launch
(cq_pool_timing's host time per launch), which is hipLaunchKernel alone.
Paths (INT4 int4gemv_cdna4 at N x K, then FP16 gemv_cdna4 and torch.mv):
  forward_into       the public call (the fast path of csrc/cq_pyfast.cpp)
  forward            the same, allocating the output
  forward_grouped    three problems of the shape in one grouped launch
  checked path       variant lookup, the metadata checks in the reference's
                     order and the ctypes launch (what forward_into runs
                     when the fast path declines)
  cq_int4gemv        the raw C entry point through ctypes
  cq_launch_prepared a prepared launch through ctypes
  torch.mv fp16      for scale: torch's own GEMV call on the same shape
"""
from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import sys
import time

import torch


def _sleep_cycles_per_us() -> float:
    """Rate of torch.cuda._sleep's cycle count, from the fastest of three
    timed waits (the first is a warm-up of the kernel itself)."""
    rates = []
    for _ in range(4):
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(4_000_000)
        e1.record()
        torch.cuda.synchronize()
        rates.append(4_000_000 / (e0.elapsed_time(e1) * 1e3))
    return max(rates[1:])


MAX_WAIT_US = 2_000_000.0


def _guess_us(fn, n: int = 50) -> float:
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        fn()
    us = (time.perf_counter() - t0) / n * 1e6
    torch.cuda.synchronize()
    return us


def _busy_loop(fn, calls: int, wait_us: float, cycles_per_us: float):
    """Host µs per call of one loop of `calls` calls issued behind an
    on-device wait of `wait_us`, or None if the wait ended before the loop
    did (the GPU was not busy throughout)."""
    torch.cuda._sleep(int(wait_us * cycles_per_us))
    done = torch.cuda.Event()
    done.record()
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    t1 = time.perf_counter()
    still = not done.query()
    torch.cuda.synchronize()
    return (t1 - t0) / calls * 1e6 if still else None


def host_us_per_call(paths: dict, calls: int, reps: int, cycles_per_us: float) -> dict:
    """Median host µs per call of every path in `paths` (name -> fn).  The
    paths are measured in `reps` interleaved rounds (one loop of each per
    round), so a drift of the host's speed during the run (clock ramp,
    other load) spreads over all of them instead of favouring the last.  A
    loop that outran its wait is repeated with the wait doubled (up to
    MAX_WAIT_US, at most 3 tries per round)."""
    wait = {name: max(20_000.0, 4.0 * _guess_us(fn) * calls) for name, fn in paths.items()}
    vals: dict = {name: [] for name in paths}
    loops = dict.fromkeys(paths, 0)
    for _ in range(reps):
        for name, fn in paths.items():
            for _try in range(3):
                loops[name] += 1
                us = _busy_loop(fn, calls, wait[name], cycles_per_us)
                if us is not None:
                    vals[name].append(us)
                    break
                wait[name] = min(MAX_WAIT_US, 2.0 * wait[name])
    return {name: {"us": round(statistics.median(v), 3) if v else None,
                   "samples": len(v), "loops": loops[name]}
            for name, v in vals.items()}


def run(n: int = 4096, k: int = 4096, calls: int = 1000, reps: int = 7) -> dict:
    from .. import _capi
    from ..build import build
    from ..operators.int4gemv import device_random_set

    ext4, extg = build("int4gemv"), build("gemv")
    W, s, x, out = device_random_set(n, k, 1)
    v = "int4gemv_cdna4"
    Wg = (torch.randn(n, k, device="cuda") * 0.02).half()
    xg = torch.randn(k, device="cuda").half()
    og = torch.empty(n, dtype=torch.float16, device="cuda")
    lib = _capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (W.data_ptr(), s.data_ptr(), x.data_ptr(), out.data_ptr())
    vb = v.encode()
    prepared = _capi.CqPrepared()     # must outlive every call through `addr`
    _capi.check(lib.cq_prepare(_capi.CQ_OP_INT4GEMV, vb, *ptrs, n, k,
                               ctypes.byref(prepared)), "cq_prepare")
    addr = ctypes.addressof(prepared)

    group = [(W, s, x, out)] + [device_random_set(n, k, 2 + i) for i in range(2)]

    def checked():
        ext4._lookup(v)
        ext4._validate_inputs(W, s, x)
        ext4._validate_out(W, out)
        ext4._launch(v, W, s, x, out)

    paths = {
        "forward_into": lambda: ext4.forward_into(v, W, s, x, out),
        "forward": lambda: ext4.forward(v, W, s, x),
        "forward_grouped (3 problems)": lambda: ext4.forward_grouped(v, group),
        "checked path": checked,
        "cq_int4gemv (ctypes)": lambda: lib.cq_int4gemv(vb, *ptrs, n, k, stream),
        "cq_launch_prepared (ctypes)": lambda: lib.cq_launch_prepared(addr, stream),
        "gemv forward_into fp16": lambda: extg.forward_into("gemv_cdna4", Wg, xg, og),
        "torch.mv fp16": lambda: torch.mv(Wg, xg),
    }
    cpu = _sleep_cycles_per_us()
    res = {"n": n, "k": k, "calls": calls, "reps": reps,
           "device": torch.cuda.get_device_name(0),
           "library": _capi.version()}
    # warm the host (clock ramp, caches) with a second of every path
    t_end = time.perf_counter() + 1.0
    while time.perf_counter() < t_end:
        for fn in paths.values():
            fn()
    torch.cuda.synchronize()
    # the floor under every path: the library's own C loop enqueueing the
    # same launch behind an on-device wait (hipLaunchKernel and nothing else),
    # measured as one more interleaved path
    from ..ext import pool_timing, prefill_delay_us
    native: list = []

    def native_loop():
        r = pool_timing("int4gemv", v, [(W, s, x, out)], warmup=0, n_launches=calls,
                        per_kernel=False, delay_us=prefill_delay_us(calls))
        native.append(r["host_us"] / calls)

    def statuses_ok() -> None:
        # the raw entry points report failure only through their status
        _capi.check(lib.cq_int4gemv(vb, *ptrs, n, k, stream), "cq_int4gemv")
        _capi.check(lib.cq_launch_prepared(addr, stream), "cq_launch_prepared")
        torch.cuda.synchronize()

    statuses_ok()
    res["host_us_per_call"] = {}
    for _ in range(reps):
        native_loop()
        r = host_us_per_call(paths, calls, 1, cpu)
        for name, one in r.items():
            agg = res["host_us_per_call"].setdefault(name, {"vals": [], "samples": 0, "loops": 0})
            if one["us"] is not None:
                agg["vals"].append(one["us"])
            agg["samples"] += one["samples"]
            agg["loops"] += one["loops"]
    statuses_ok()
    res["native_enqueue_us_per_launch"] = round(statistics.median(native), 3)
    print(f"{'native C enqueue (floor)':<30} {res['native_enqueue_us_per_launch']} us", flush=True)
    for name, agg in res["host_us_per_call"].items():
        vals = agg.pop("vals")
        agg["us"] = round(statistics.median(vals), 3) if vals else None
        print(f"{name:<30} {agg['us']} us  ({agg['samples']} of {agg['loops']} loops ended "
              "with the GPU still busy)", flush=True)
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--k", type=int, default=4096)
    ap.add_argument("--calls", type=int, default=1000)
    ap.add_argument("--reps", type=int, default=7)
    ap.add_argument("--json", default=None)
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("api_cost: no GPU visible", file=sys.stderr)
        return 1
    res = run(a.n, a.k, a.calls, a.reps)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
