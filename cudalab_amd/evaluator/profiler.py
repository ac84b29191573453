"""rocprofv3 adapter: per-variant kernel profiles on MI355X.

Role of `cudalab/evaluator/profiler.py` (which ran Nsight Compute over a
small driver program and turned its CSV into a JSON summary) on ROCm:

* the operator adapter supplies the driver source
  (`op.profile_driver_source(variant, M, K)`, a few launches of one
  variant) and the kernel-name pattern (`op.kernel_regex`), as in the
  reference (:66-88);
* the driver runs as a child process under `rocprofv3 --kernel-trace
  --stats -f csv`; the per-dispatch device durations of the matching
  kernels become the summary (count, median, mean, min, max, and the
  algorithmic bandwidth at the median);
* hardware counters (`counters`: groups of PMC names) are collected in
  passes of their own, one `rocprofv3 --pmc` run per group, never combined
  with a trace, each under a hard time limit.  A group must fit the
  counter blocks of one pass (at most 8 SQ, 4 TCC -- FETCH_SIZE takes 3,
  WRITE_SIZE 2 --, 4 TCP, 2 TA, 2 TD, 2 GRBM);
* a metric that cannot be read is null, never invented; the tools' own
  output is kept in the run directory's raw/ folder.

The program after `--` is the Python interpreter itself (no shell, env or
launcher in between).
"""
from __future__ import annotations

import json
import os
import re
import shutil
import statistics
import subprocess
import sys
import tempfile
from pathlib import Path

from .gpu import now_iso
from .rocprof_summary import counter_values, dispatch_times


def rocprof_path() -> str | None:
    p = shutil.which("rocprofv3")
    if p is None and Path("/opt/rocm/bin/rocprofv3").exists():
        p = "/opt/rocm/bin/rocprofv3"
    return p


def rocprof_version() -> str:
    tool = rocprof_path()
    if tool is None:
        return "unavailable"
    try:
        r = subprocess.run([tool, "--version"], capture_output=True, text=True,
                           timeout=60)
        m = re.search(r"(\d+\.\d+\.\d+)", r.stdout + r.stderr)
        return m.group(1) if m else "unknown"
    except Exception:  # noqa: BLE001
        return "unknown"


def _run(cmd: list[str], cwd: Path, log: Path, timeout: float) -> int:
    env = dict(os.environ, TMPDIR=str(cwd))
    try:
        r = subprocess.run(cmd, cwd=cwd, env=env, capture_output=True,
                           text=True, timeout=timeout)
        log.write_text(r.stdout + "\n--- stderr ---\n" + r.stderr)
        return r.returncode
    except subprocess.TimeoutExpired as e:
        out = e.stdout.decode() if isinstance(e.stdout, bytes) else (e.stdout or "")
        log.write_text(out + f"\n--- killed after {timeout} s ---\n")
        return -9


def _stats_us(ns: list[int]) -> dict:
    us = sorted(v / 1e3 for v in ns)
    return {"n": len(us), "median_us": round(us[len(us) // 2], 3),
            "mean_us": round(statistics.fmean(us), 3),
            "min_us": round(us[0], 3), "max_us": round(us[-1], 3)}


def profile_variant(op, variant: str, M: int, K: int,
                    out_dir: Path | None = None,
                    counters: list[list[str]] | None = None,
                    timeout: float = 300.0) -> dict:
    """Profile one variant at (M, K) and return (and save as
    out_dir/summary.json) its summary.  `out_dir` defaults to a fresh
    temporary directory."""
    tool = rocprof_path()
    out_dir = Path(out_dir or tempfile.mkdtemp(prefix="cq_rocprof_"))
    raw = out_dir / "raw"
    raw.mkdir(parents=True, exist_ok=True)
    driver = raw / "driver.py"
    driver.write_text(op.profile_driver_source(variant, M, K))
    summary: dict = {
        "tool": "rocprofv3", "version": rocprof_version(),
        "operator": op.name, "variant": variant, "shape": [M, K],
        "kernel_regex": op.kernel_regex, "generated": now_iso(),
        "raw_dir": str(raw), "kernels": [], "kernel_duration_us": None,
        "algorithmic_bw_gbps": None, "counters": {}, "errors": [],
    }
    if tool is None:
        summary["errors"].append("rocprofv3 not found")
        return _save(out_dir, summary)

    trace = raw / "trace"
    cmd = [tool, "--kernel-trace", "--stats", "-f", "csv", "-d", str(trace),
           "-o", "prof", "--", sys.executable, str(driver)]
    summary["trace_command"] = " ".join(cmd)
    rc = _run(cmd, raw, raw / "trace.log", timeout)
    summary["trace_returncode"] = rc
    pat = re.compile(op.kernel_regex)
    by = dispatch_times(trace) if trace.exists() else {}
    hits = {name: v for name, v in by.items() if pat.search(name)}
    for name, v in sorted(hits.items(), key=lambda kv: -len(kv[1])):
        summary["kernels"].append({"name": name,
                                   **_stats_us([e - s for s, e in v])})
    if summary["kernels"]:
        main = summary["kernels"][0]
        summary["kernel_duration_us"] = main["median_us"]
        nbytes = op.algorithmic_bytes(M, K, 2)
        summary["algorithmic_bytes"] = nbytes
        summary["algorithmic_bw_gbps"] = round(nbytes / main["median_us"] / 1e3, 1)
    elif rc != 0:
        summary["errors"].append(f"trace run exited with {rc} (see raw/trace.log)")
    else:
        summary["errors"].append(f"no dispatch matched {op.kernel_regex!r}")

    for i, group in enumerate(counters or []):
        d = raw / f"pmc{i}"
        cmd = [tool, "--pmc", *group, "-f", "csv", "-d", str(d), "-o", "prof",
               "--", sys.executable, str(driver)]
        rc = _run(cmd, raw, raw / f"pmc{i}.log", min(timeout, 120.0))
        for c in group:
            vals = []
            if d.exists():
                for name, v in counter_values(d, c).items():
                    if pat.search(name):
                        vals.extend(v)
            summary["counters"][c] = statistics.median(vals) if vals else None
        if rc != 0:
            summary["errors"].append(f"pmc pass {i} {group} exited with {rc}")
    return _save(out_dir, summary)


def _save(out_dir: Path, summary: dict) -> dict:
    (out_dir / "summary.json").write_text(json.dumps(summary, indent=2))
    return summary
