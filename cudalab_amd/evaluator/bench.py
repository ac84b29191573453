"""Timing pools and the paired A/B engine of the GEMV path.

Drop-in for `cudalab/evaluator/bench.py` (harness paired-streaming-v2.3):
`BenchPool` (:197-246), `measure_block` (:259-309), `bench_pair`
(:328-561), `bench_matrix` (:564-733), `analyze_shape_winners`
(:736-768), `save_record` (:763-768) and `time_call` (:772-794).  The
methodology is kept: rounds as the unit of inference, parent and candidate
adjacent within a round on the same tensors with the order alternating
(pair) or rotating (matrix), symmetric sample and cross-block guards with
raw and filtered tracks, up to 3 retries of an invalid round, no clock
sampling inside a round, and GPU state snapshots (amd-smi) only before
and after a run.

What is MI355X-specific:

* Caliber.  A timed sample is `batch` back-to-back launches between two
  HIP events.  With caliber "native" (the default here) the launches come
  from the library's C loop over the pool (cq_pool_timing), queued behind
  an on-device wait so that the host is ahead of the GPU for the whole
  sample; with "api" they go through the Python extension object as in
  the reference.  The GEMVs take 3-5 us on MI355X, less than one
  Python-boundary call, so the "api" caliber times the host, not the
  kernels.
* Cache.  "streaming" pools are HBM-cold: distinct full (W, scale, x, out)
  sets totalling more than 512 MiB, twice the 256 MiB MALL, rotated launch
  by launch (the reference rotated only x/out over a shared W, which stays
  MALL-resident on MI355X; that mode is kept as "x-rotate").

Modes of a pool:
  "hot"        one set, back-to-back launches (W resident in MALL / L2).
  "streaming"  the HBM-cold rotating pool of distinct sets.
  "x-rotate"   only x/out rotate, W shared (the reference's "streaming").
"""
from __future__ import annotations

import json
import statistics
import time
from pathlib import Path
from dataclasses import dataclass, field
from typing import Callable, Optional

import torch

from . import stats as _stats
from .experiment import classify_cell
from .gpu import gpu_state, now_iso
from .stats import (CROSSBLOCK_FACTOR, CROSSBLOCK_WARMUP, SPIKE_FACTOR,  # noqa: F401
                    SPIKE_WINDOW, apply_spike_guard, block_stats,
                    crossblock_flag)

HARNESS_VERSION = "paired-streaming-v2.3"
WARMUP = 150        # untimed launches before a block (minimum count)
WARMUP_MS = 300.0   # ... and minimum wall time of that burn
ITERS = 100         # timed samples per block
BATCH = 32          # back-to-back launches per sample
POOL_SIZE = 16      # x/out buffers of an "x-rotate" pool
SEED = 1234         # input generator seed
COLD_POOL_BYTES = 512 * 1024 * 1024   # streaming pool floor (> 256 MB MALL)
MODES = ("hot", "streaming", "x-rotate")
CALIBERS = ("native", "api")
ROUNDS = 9          # independent rounds per record
MAX_RETRIES = 3     # retries of an invalid round
MIN_VALID_ROUNDS = 5
MIN_CLEAN_SAMPLES = 50   # accepted samples a block needs for a valid round
DVFS_TOL = 0.05     # clock tolerance of the v0.2 records (no round samples clocks)
LLC_BYTES = 256 * 1024 * 1024   # MI355X MALL (last-level cache)


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
    op: str = ""        # operator id of the native loop ("int4gemv", ...)

    def __post_init__(self):
        if self.mode not in MODES:
            raise ValueError(f"unknown cache mode: {self.mode!r} "
                             f"(expected one of {MODES})")
        if self.mode == "hot":
            if len(self.xs) != 1 or len(self.outs) != 1:
                raise ValueError("hot mode needs exactly one x/out buffer")
        elif len(self.xs) != self.pool_size or len(self.outs) != self.pool_size:
            raise ValueError("a rotating pool needs pool_size x/out buffers")


def _api_sampler(pool: BenchPool, ext, variant: str):
    """k launches through the Python extension object; returns window us."""
    n = 1 if pool.mode == "hot" else pool.pool_size
    idx = [0]
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)

    def run(k: int, timed: bool) -> float:
        if timed:
            start.record()
        for _ in range(k):
            pool.launch(ext, variant, idx[0])
            idx[0] = (idx[0] + 1) % n
        if not timed:
            return 0.0
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e3
    return run


def _native_sampler(pool: BenchPool, variant: str):
    """k launches from the library's C loop (cq_pool_timing) over the
    pool's sets, continuing the rotation between calls; returns window us
    (events on the current stream around the k launches).  A timed sample
    is queued behind an on-device wait, so that the host has enqueued all k
    launches before the GPU reaches them and the sample times the GPU, not
    the host's submission rate (2.5-3.5 us per launch, as long as a short
    GEMV)."""
    from ..ext import pool_timing, prefill_delay_us
    if not pool.sets or not pool.op:
        raise ValueError("the native caliber needs a pool with sets and op")
    sets = pool.sets
    n = len(sets)
    off = [0]

    def run(k: int, timed: bool) -> float:
        o = off[0]
        rot = sets[o:] + sets[:o]
        r = pool_timing(pool.op, variant, rot, warmup=0, n_launches=k,
                        per_kernel=False,
                        delay_us=prefill_delay_us(k) if timed else 0.0)
        off[0] = (o + k) % n
        return r["total_us"]
    return run


def measure_block(pool: BenchPool, ext, variant: str, warmup: int = WARMUP,
                  iters: int = ITERS, batch: int = BATCH,
                  warmup_ms: float = WARMUP_MS,
                  spike_factor: float = SPIKE_FACTOR,
                  caliber: str = "native") -> dict:
    """One block: per-launch time (us) of `variant` in `iters` samples of
    `batch` back-to-back launches, after a burn of >= warmup launches and
    >= warmup_ms of wall time (a GPU coming out of idle runs slow for a
    while).  Returns block_stats of the samples (raw and filtered tracks)
    plus min_us / mean_us of the raw samples and the caliber."""
    if caliber not in CALIBERS:
        raise ValueError(f"unknown caliber {caliber!r} (expected one of {CALIBERS})")
    run = (_native_sampler(pool, variant) if caliber == "native"
           else _api_sampler(pool, ext, variant))
    t0 = time.perf_counter()
    done = 0
    while done < warmup or (time.perf_counter() - t0) * 1e3 < warmup_ms:
        run(max(1, min(warmup, 64)), timed=False)
        done += max(1, min(warmup, 64))
    torch.cuda.synchronize()
    raw = [run(batch, timed=True) / batch for _ in range(iters)]
    out = block_stats(raw, spike_factor=spike_factor, window=SPIKE_WINDOW)
    out["min_us"] = min(raw) if raw else None
    out["mean_us"] = statistics.fmean(raw) if raw else None
    out["caliber"] = caliber
    return out


def _require_normal_variant(op, ext, v: str) -> None:
    """Only dispatchable variants (or their reference-name aliases) enter
    a benchmark; a quarantined one is refused with the reason."""
    if v in op.variants(ext) or v in getattr(ext, "aliases", dict)():
        return
    if v in op.unsafe_variants(ext):
        raise ValueError(f"variant {v!r} is quarantined (NOT_FOR_NORMAL_DISPATCH) "
                         "and cannot enter a normal benchmark; an explicit "
                         f"ext.forward({v!r}, ...) call remains possible")
    raise ValueError(f"unknown variant {v!r}")


def _environment_guard() -> dict:
    return {
        "method": ("symmetric guards: a sample outside [ref/1.5, ref*1.5] of "
                   "the median of the last 50 accepted samples is rejected; a "
                   "block whose filtered median is outside [run/1.15, "
                   "run*1.15] of the variant's running block median "
                   "invalidates the round (after 3 blocks); parent and "
                   "candidate use the same rule and thresholds"),
        "symmetric": True,
        "spike_factor": SPIKE_FACTOR,
        "spike_window": SPIKE_WINDOW,
        "crossblock_factor": CROSSBLOCK_FACTOR,
        "crossblock_warmup": CROSSBLOCK_WARMUP,
        "min_accepted_samples": MIN_CLEAN_SAMPLES,
        "filter_sensitive_log_delta": round(_stats.FILTER_LOG_DELTA, 6),
        "raw_and_filtered_recorded": True,
    }


def _clock_policy(max_retries: int) -> dict:
    return {"sm_clock_rel_tolerance": DVFS_TOL,
            "min_valid_rounds": MIN_VALID_ROUNDS,
            "max_retries": max_retries,
            "warmup_ms": WARMUP_MS,
            "spike_factor": SPIKE_FACTOR,
            "spike_window": SPIKE_WINDOW,
            "min_clean_samples": MIN_CLEAN_SAMPLES,
            "crossblock_factor": CROSSBLOCK_FACTOR,
            "crossblock_warmup": CROSSBLOCK_WARMUP,
            "note": ("no clock sampling inside a round (a query leaves the GPU "
                     "idle and perturbs what follows); drift between A and B "
                     "is caught by the symmetric cross-block guard; amd-smi "
                     "snapshots before and after the run")}


def _record_head(op, M: int, K: int, dtype, mode: str, seed: int, warmup: int,
                 iters: int, batch: int, max_retries: int, pool: BenchPool,
                 caliber: str) -> dict:
    return {
        "harness": HARNESS_VERSION,
        "platform": "MI355X (gfx950)",
        "caliber": caliber,
        "operator": op.name,
        "shape": [M, K],
        "dtype": str(dtype).split(".")[-1],
        "cache_mode": mode,
        "seed": seed,
        "warmup": warmup, "iters": iters, "batch": batch,
        "pool": {"pool_size": pool.pool_size,
                 "working_set_bytes": pool.working_set_bytes,
                 "working_set_gt_llc": pool.working_set_bytes > LLC_BYTES,
                 "shared_bytes": pool.shared_bytes,
                 "pool_extra": pool.pool_extra},
        "clock_policy": _clock_policy(max_retries),
        "environment_guard": _environment_guard(),
        "generated": now_iso(),
    }


def _round_validity(blocks: dict, cross: dict) -> tuple[bool, str | None]:
    if not all(b["n_clean"] >= MIN_CLEAN_SAMPLES for b in blocks.values()):
        return False, "INVALID_SPIKES"
    if any(c["flagged"] for c in cross.values()):
        return False, "INVALID_CROSSBLOCK"
    return True, None


def bench_pair(op, ext, parent: str, candidate: str, M: int, K: int,
               dtype: torch.dtype = torch.float16, mode: str = "streaming",
               rounds: int = ROUNDS, warmup: int = WARMUP, iters: int = ITERS,
               batch: int = BATCH, max_retries: int = MAX_RETRIES,
               seed: int = SEED, caliber: str = "native") -> dict:
    """Paired A/B: in every round parent and candidate are measured back
    to back on the same pool, parent first in even rounds and second in
    odd ones.  The record holds every round (raw and filtered), the paired
    statistics of the valid rounds and the filter-sensitivity verdict;
    decide it with decision.decide_v2 + apply_filter_gate."""
    if mode not in MODES:
        raise ValueError(f"unknown cache mode: {mode!r} (expected one of {MODES})")
    for v in (parent, candidate):
        _require_normal_variant(op, ext, v)
    pool = op.make_bench_pool(M, K, dtype, mode, seed=seed, pool_size=POOL_SIZE)
    algo = op.algorithmic_bytes(M, K, pool.element_size)
    rec = _record_head(op, M, K, dtype, mode, seed, warmup, iters, batch,
                       max_retries, pool, caliber)
    rec.update({"parent": parent, "candidate": candidate})
    rec["gpu_state_before"] = gpu_state()
    hist: dict[str, list[float]] = {parent: [], candidate: []}
    rounds_out: list[dict] = []
    for slot in range(rounds):
        order = [parent, candidate] if slot % 2 == 0 else [candidate, parent]
        res: dict = {}
        for attempt in range(max_retries + 1):
            blocks = {v: measure_block(pool, ext, v, warmup, iters, batch,
                                       caliber=caliber) for v in order}
            cross = {v: crossblock_flag(hist[v], blocks[v]["median_us"])
                     for v in (parent, candidate)}
            ok, why = _round_validity(blocks, cross)
            bp, bc = blocks[parent], blocks[candidate]
            tp, tc = bp["median_us"], bc["median_us"]
            rp, rc = bp["raw_median_us"], bc["raw_median_us"]
            res = {
                "round": slot + 1, "order": order, "retries": attempt,
                "parent_us": round(tp, 3) if tp else None,
                "candidate_us": round(tc, 3) if tc else None,
                "speedup": round(tp / tc, 6) if tp and tc else None,
                "parent_raw_us": round(rp, 3) if rp else None,
                "candidate_raw_us": round(rc, 3) if rc else None,
                "raw_speedup": round(rp / rc, 6) if rp and rc else None,
                "valid": ok, "invalid_reason": why,
                "samples": {"parent": bp, "candidate": bc},
                "crossblock": cross,
            }
            if ok:
                break
        rounds_out.append(res)

    valid = [r for r in rounds_out if r["valid"]]
    speedups = _stats.paired_speedups([r["parent_us"] for r in valid],
                                      [r["candidate_us"] for r in valid])
    s = _stats.summarize(speedups)
    ci95 = _stats.bootstrap_ci(speedups)
    p_med = statistics.median([r["parent_us"] for r in valid]) if valid else None
    c_med = statistics.median([r["candidate_us"] for r in valid]) if valid else None
    raw_p = [r["parent_raw_us"] for r in valid if r["parent_raw_us"] is not None]
    raw_c = [r["candidate_raw_us"] for r in valid if r["candidate_raw_us"] is not None]
    if raw_p and len(raw_p) == len(raw_c):
        raw_speedups = _stats.paired_speedups(raw_p, raw_c)
        raw_speedup = _stats.summarize(raw_speedups)["median"]
        ci95_raw = _stats.bootstrap_ci(raw_speedups)
    else:
        raw_speedup, ci95_raw = None, None
    raw_p_med = statistics.median(raw_p) if raw_p else None
    raw_c_med = statistics.median(raw_c) if raw_c else None
    fs, fs_why = _stats.filter_sensitive(raw_speedup, s["median"])
    n_invalid = len(rounds_out) - len(valid)
    n_invalid_env = sum(1 for r in rounds_out if not r["valid"]
                        and r["invalid_reason"] != "INVALID_SPIKES")

    def r3(v):
        return round(v, 3) if v else None

    rec.update({
        "n_rounds": len(rounds_out),
        "valid_rounds": len(valid),
        "invalid_environment_rounds": n_invalid,
        "invalid_environment_only_rounds": n_invalid_env,
        "invalid_dvfs_rounds": n_invalid,
        "invalid_dvfs_only_rounds": n_invalid_env,
        "invalid_spikes_rounds": sum(1 for r in rounds_out
                                     if r["invalid_reason"] == "INVALID_SPIKES"),
        "invalid_crossblock_rounds": sum(1 for r in rounds_out
                                         if r["invalid_reason"] == "INVALID_CROSSBLOCK"),
        "rounds": rounds_out,
        "speedups": speedups,
        "median_speedup": s["median"],
        "mean_speedup": s["mean"],
        "min_speedup": s["min"],
        "max_speedup": s["max"],
        "faster_rounds": f"{s['faster_count']}/{s['n']}",
        "bootstrap_ci_95": ci95,
        "bootstrap": {"n_boot": _stats.BOOTSTRAP_N, "seed": _stats.BOOTSTRAP_SEED,
                      "statistic": "median"},
        "parent_median_us": r3(p_med),
        "candidate_median_us": r3(c_med),
        "raw_speedup": raw_speedup,
        "filtered_speedup": s["median"],
        "filter_sensitive": fs,
        "filter_sensitive_reason": fs_why,
        "raw": {"parent_median_us": r3(raw_p_med),
                "candidate_median_us": r3(raw_c_med),
                "speedup": raw_speedup, "bootstrap_ci_95": ci95_raw},
        "filtered": {"parent_median_us": r3(p_med),
                     "candidate_median_us": r3(c_med),
                     "speedup": s["median"], "bootstrap_ci_95": ci95},
        "rejected_samples": {
            "fast": sum(r["samples"][k]["n_rejected_fast"] for r in rounds_out
                        for k in ("parent", "candidate")),
            "slow": sum(r["samples"][k]["n_rejected_slow"] for r in rounds_out
                        for k in ("parent", "candidate"))},
        "algorithmic_bytes": algo,
        "algorithmic_bw_gbps_parent":
            round(algo / (p_med * 1e-6) / 1e9, 1) if p_med else None,
        "algorithmic_bw_gbps_candidate":
            round(algo / (c_med * 1e-6) / 1e9, 1) if c_med else None,
    })
    rec["gpu_state_after"] = gpu_state()
    del pool
    torch.cuda.empty_cache()
    return rec


def bench_matrix(op, ext, variants: list[str], M: int, K: int,
                 dtype: torch.dtype = torch.float16, mode: str = "streaming",
                 rounds: int = ROUNDS, warmup: int = WARMUP, iters: int = ITERS,
                 batch: int = BATCH, max_retries: int = MAX_RETRIES,
                 seed: int = SEED, caliber: str = "native") -> dict:
    """Round-robin matrix: every round measures all variants back to back
    on the same pool, the starting variant rotating by round.  Classify the
    record with analyze_shape_winners."""
    if mode not in MODES:
        raise ValueError(f"unknown cache mode: {mode!r} (expected one of {MODES})")
    for v in variants:
        _require_normal_variant(op, ext, v)
    pool = op.make_bench_pool(M, K, dtype, mode, seed=seed, pool_size=POOL_SIZE)
    algo = op.algorithmic_bytes(M, K, pool.element_size)
    rec = _record_head(op, M, K, dtype, mode, seed, warmup, iters, batch,
                       max_retries, pool, caliber)
    rec["gpu_state_before"] = gpu_state()
    n = len(variants)
    hist: dict[str, list[float]] = {v: [] for v in variants}
    rounds_out: list[dict] = []
    for slot in range(rounds):
        order = variants[slot % n:] + variants[:slot % n]
        res: dict = {}
        for attempt in range(max_retries + 1):
            blocks = {v: measure_block(pool, ext, v, warmup, iters, batch,
                                       caliber=caliber) for v in order}
            cross = {v: crossblock_flag(hist[v], blocks[v]["median_us"])
                     for v in order}
            ok, why = _round_validity(blocks, cross)
            res = {
                "round": slot + 1, "order": order, "retries": attempt,
                "valid": ok, "invalid_reason": why,
                "us": {v: round(blocks[v]["median_us"], 3) for v in order},
                "us_raw": {v: (round(blocks[v]["raw_median_us"], 3)
                               if blocks[v]["raw_median_us"] else None)
                           for v in order},
                "samples": blocks,
                "crossblock": cross,
            }
            if ok:
                break
        rounds_out.append(res)

    valid = [r for r in rounds_out if r["valid"]]
    per_variant = {}
    for v in variants:
        meds = [r["us"][v] for r in valid]
        raws = [r["us_raw"][v] for r in valid if r["us_raw"].get(v) is not None]
        med = statistics.median(meds) if meds else None
        raw_med = statistics.median(raws) if raws else None
        per_variant[v] = {
            "round_medians_us": meds,
            "median_us": round(med, 3) if med else None,
            "round_raw_medians_us": [r["us_raw"][v] for r in valid],
            "raw_median_us": round(raw_med, 3) if raw_med else None,
            "algorithmic_bw_gbps": round(algo / (med * 1e-6) / 1e9, 1) if med else None,
            "n_valid_rounds": len(meds),
        }
    cell = classify_cell(variants, rounds_out)
    rec.update({
        "variants": variants,
        "n_rounds": len(rounds_out),
        "valid_rounds": len(valid),
        "invalid_environment_rounds": len(rounds_out) - len(valid),
        "invalid_dvfs_rounds": len(rounds_out) - len(valid),
        "invalid_spikes_rounds": sum(1 for r in rounds_out
                                     if r["invalid_reason"] == "INVALID_SPIKES"),
        "invalid_crossblock_rounds": sum(1 for r in rounds_out
                                         if r["invalid_reason"] == "INVALID_CROSSBLOCK"),
        "winner_raw": cell.get("winner_raw"),
        "filter_sensitive": cell.get("filter_sensitive", False),
        "filter_sensitive_reason": cell.get("filter_sensitive_reason"),
        "rejected_samples": {
            "fast": sum(b["n_rejected_fast"] for r in rounds_out
                        for b in r["samples"].values()),
            "slow": sum(b["n_rejected_slow"] for r in rounds_out
                        for b in r["samples"].values())},
        "rounds": rounds_out,
        "per_variant": per_variant,
        "algorithmic_bytes": algo,
    })
    rec["gpu_state_after"] = gpu_state()
    del pool
    torch.cuda.empty_cache()
    return rec


def analyze_shape_winners(records: list[dict]) -> list[dict]:
    """Per-cell winners of matrix records, each classified by
    experiment.classify_cell (the single source of the statistics)."""
    return [{"shape": r["shape"], "dtype": r["dtype"],
             "cache_mode": r["cache_mode"],
             **classify_cell(r["variants"], r["rounds"])} for r in records]


def save_record(record: dict, out_dir: Path, tag: str = "") -> Path:
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    path = out_dir / f"{tag}.json"
    path.write_text(json.dumps(record, indent=2, ensure_ascii=False))
    return path


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
