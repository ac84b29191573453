"""Timing pool and the API-path timing loop.

Drop-in for the parts of `cudalab/evaluator/bench.py` that define the
timing caliber of the GEMV path: `BenchPool` (:197-246), `measure_block`
(:259-309) and `time_call` (:772-794), plus the shared constants.  The
paired A/B decision machinery of that file (bench_pair, bench_matrix, the
spike and cross-block guards) is not part of this path and is not here;
`measure_block` reports raw-sample statistics.

Modes of a pool:
  "hot"        one (W, scale, x, out) set, back-to-back launches: on MI355X
               W stays in the 256 MB MALL / L2.
  "streaming"  HBM-cold: a rotating pool of distinct full sets whose total
               exceeds 512 MiB, so each launch reads W from HBM.
  "x-rotate"   the reference's "streaming": only x/out rotate and W is
               shared (cudalab/operators/int4gemv.py:186-236); on MI355X W
               is MALL-resident, so this is reported as context only.
"""
from __future__ import annotations

import statistics
import time
from dataclasses import dataclass, field
from typing import Callable, Optional

import torch

WARMUP = 150        # untimed launches before a block (minimum count)
WARMUP_MS = 300.0   # ... and minimum wall time of that burn
ITERS = 100         # timed samples per block
BATCH = 32          # back-to-back launches per sample
POOL_SIZE = 16      # x/out buffers of an "x-rotate" pool
SEED = 1234         # input generator seed
COLD_POOL_BYTES = 512 * 1024 * 1024   # streaming pool floor (> 256 MB MALL)
MODES = ("hot", "streaming", "x-rotate")


@dataclass
class BenchPool:
    """Preallocated timing tensors: nothing is allocated, generated or
    copied inside a timed region.  `launch(ext, variant, i)` performs one
    timed call on set/buffer i (i is always 0 in hot mode)."""
    xs: list
    outs: list
    pool_size: int
    working_set_bytes: int
    element_size: int
    mode: str
    launch: Callable = field(repr=False)
    positions: Optional[list] = None
    shared: dict = field(default_factory=dict, repr=False)
    shared_bytes: int = 0
    pool_extra: dict = field(default_factory=dict)
    sets: list = field(default_factory=list, repr=False)

    def __post_init__(self):
        if self.mode not in MODES:
            raise ValueError(f"unknown cache mode: {self.mode!r} "
                             f"(expected one of {MODES})")
        if self.mode == "hot":
            if len(self.xs) != 1 or len(self.outs) != 1:
                raise ValueError("hot mode needs exactly one x/out buffer")
        elif len(self.xs) != self.pool_size or len(self.outs) != self.pool_size:
            raise ValueError("a rotating pool needs pool_size x/out buffers")


def measure_block(pool: BenchPool, ext, variant: str, warmup: int = WARMUP,
                  iters: int = ITERS, batch: int = BATCH,
                  warmup_ms: float = WARMUP_MS) -> dict:
    """API-path caliber: per-launch time (us) through the Python boundary.

    Burn >= warmup launches and >= warmup_ms of wall time, then `iters`
    samples of `batch` back-to-back launches between torch events (the
    launches rotate through the pool's buffers/sets)."""
    n = 1 if pool.mode == "hot" else pool.pool_size
    idx = [0]

    def one():
        i = idx[0]
        pool.launch(ext, variant, i)
        idx[0] = (i + 1) % n

    t0 = time.perf_counter()
    done = 0
    while done < warmup or (time.perf_counter() - t0) * 1e3 < warmup_ms:
        one()
        done += 1
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    raw: list[float] = []
    for _ in range(iters):
        start.record()
        for _ in range(batch):
            one()
        stop.record()
        torch.cuda.synchronize()
        raw.append(start.elapsed_time(stop) * 1e3 / batch)
    return {
        "median_us": statistics.median(raw),
        "raw_median_us": statistics.median(raw),
        "min_us": min(raw),
        "mean_us": statistics.fmean(raw),
        "n_raw": len(raw),
        "raw_samples_us": [round(v, 3) for v in raw],
    }


def time_call(fn: Callable, warmup: int = 100, iters: int = 200,
              batch: int = 32) -> dict:
    """Generic timing helper with the same batching as measure_block."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    times: list[float] = []
    for _ in range(iters):
        start.record()
        for _ in range(batch):
            fn()
        stop.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) * 1e3 / batch)
    return {"median_us": round(statistics.median(times), 3),
            "min_us": round(min(times), 3),
            "n_samples": len(times)}


def cold_pool_sets(set_bytes: int, floor_bytes: int = COLD_POOL_BYTES,
                   minimum: int = 2) -> int:
    """Number of distinct sets whose total exceeds `floor_bytes`."""
    if set_bytes <= 0:
        raise ValueError("set_bytes must be positive")
    return max(minimum, floor_bytes // set_bytes + 1)
