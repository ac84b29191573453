"""Occupancy, memory latency and stall counters of the incumbent GEMV kernels.

Usage (on a GPU host, from the repository root):
  python -m cudalab_amd.evaluator.counters [--cases int4:4096x4096,...]
      [--out FILE] [--steps 200]

For every case (operator and shape) and every counter pass below, runs

  rocprofv3 --pmc <pass> -f csv -d <tmp>/<case>_<i> -o c -- \\
      python3 -m cudalab_amd.evaluator.sweep --modes streaming --steps S \\
      --warmup 20 --no-ceiling --ops <op> --shapes <N>x<K>

as a child process (this process never touches the GPU, so the profiler's
preloaded library initialises the GPU in the child only), each under a
90-second limit, and reduces each counter to its median over the kernel's
dispatches (rocprof_summary's counters report).  The passes respect
rocprofv3's per-block limits (8 SQ, 4 TCP, 2 TA, 2 TD, 2 GRBM counters per
run; derived metrics count their inputs).  Profiler runs serialise the
dispatches, so these are per-dispatch figures of an isolated launch.

Derived figures in the table:
  occupancy    MeanOccupancyPerCU: mean resident waves per CU over the
               dispatch (rocprofv3's accumulate(SQ_LEVEL_WAVES) / GRBM_GUI_ACTIVE / CUs)
  vmem_lat     VmemLatency: mean cycles a vector-memory instruction is in
               flight (accumulate(SQ_INST_LEVEL_VMEM) / SQ_INSTS_VMEM)
  l2_lat       TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ: mean cycles of
               one L1 -> L2 read request
  lds_lat      LdsLatency: mean cycles an LDS instruction is in flight
  lds_util     LdsUtil, % of the dispatch the LDS was active
  wait_lds     SQ_WAIT_INST_LDS / SQ_WAIT_INST_ANY: share of the waves'
               dependency waits that wait on LDS
  ta_tc        TA_ADDR_STALLED_BY_TC_CYCLES / TA_TA_BUSY: share of the
               address unit's busy cycles stalled because the L1 could not
               take more requests (memory pipeline saturated)
  td_tc        TD_TC_STALL / TD_TD_BUSY: share of the data unit's busy
               cycles waiting for L1 data
"""
from __future__ import annotations

import argparse
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
from pathlib import Path

from .rocprof_summary import counter_names, counter_values

PASSES = (
    "MeanOccupancyPerCU",
    "VmemLatency",
    "LdsLatency",
    "LdsUtil LDSBankConflict",
    "SQ_WAIT_INST_LDS SQ_WAIT_INST_ANY SQ_WAVE_CYCLES SQ_BUSY_CYCLES "
    "SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_VMEM_RD SQ_WAVES",
    "TA_ADDR_STALLED_BY_TC_CYCLES TA_TA_BUSY TCP_PENDING_STALL_CYCLES "
    "TCP_TCC_READ_REQ_LATENCY TCP_TCC_READ_REQ TD_TC_STALL TD_TD_BUSY",
)
OPS = {"int4": "int4gemv", "int8": "qgemv"}
DEFAULT_CASES = ("int4:4096x4096", "int8:4096x4096", "int4:11008x4096",
                 "int8:11008x4096", "int4:4096x11008", "int8:4096x11008",
                 "int4:4096x28672", "int8:4096x28672")


def run_case(tag: str, shape: str, steps: int, tmp: Path) -> dict[str, float]:
    """Median per dispatch of every counter of every pass, for the
    operator's GEMV kernel (LDS or K-tiled) in this case's sweep."""
    op = OPS[tag]
    out: dict[str, float] = {}
    for i, p in enumerate(PASSES, 1):
        d = tmp / f"{tag}_{shape}_{i}"
        cmd = ["rocprofv3", "--pmc", *p.split(), "-f", "csv", "-d", str(d), "-o", "c",
               "--", sys.executable, "-m", "cudalab_amd.evaluator.sweep",
               "--modes", "streaming", "--steps", str(steps), "--warmup", "20",
               "--no-ceiling", "--ops", op, "--shapes", shape]
        print(f"  {tag} {shape} pass {i}: {p}", flush=True)
        r = subprocess.run(["timeout", "-s", "KILL", "90", *cmd],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise SystemExit(f"pass {i} of {tag} {shape} failed ({r.returncode}):\n"
                             + r.stdout[-1500:])
        for c in counter_names(d):
            by = counter_values(d, c)
            hits = [k for k in by if f"{op}_lds_kernel" in k or f"{op}_tiled_kernel" in k]
            if hits:
                k = max(hits, key=lambda h: len(by[h]))
                out[c] = statistics.median(by[k])
                out["_kernel"] = k
        shutil.rmtree(d, ignore_errors=True)
    return out


def derived(c: dict[str, float]) -> dict[str, float]:
    def q(a, b):
        return c[a] / c[b] if c.get(b) else float("nan")
    return {"occupancy": c.get("MeanOccupancyPerCU", float("nan")),
            "vmem_lat": c.get("VmemLatency", float("nan")),
            "l2_lat": q("TCP_TCC_READ_REQ_LATENCY", "TCP_TCC_READ_REQ"),
            "lds_lat": c.get("LdsLatency", float("nan")),
            "lds_util": c.get("LdsUtil", float("nan")),
            "wait_lds": q("SQ_WAIT_INST_LDS", "SQ_WAIT_INST_ANY"),
            "ta_tc": q("TA_ADDR_STALLED_BY_TC_CYCLES", "TA_TA_BUSY"),
            "td_tc": q("TD_TC_STALL", "TD_TD_BUSY"),
            "valu_per_wave": q("SQ_INSTS_VALU", "SQ_WAVES"),
            "vmem_per_wave": q("SQ_INSTS_VMEM_RD", "SQ_WAVES")}


def table(res: list[tuple[str, str, dict]]) -> str:
    lines = [f"{'case':<18} {'kernel instance':<36} {'occup':>6} {'vmem_lat':>8} "
             f"{'l2_lat':>7} {'lds_lat':>7} {'lds%':>5} {'wait_lds':>8} {'ta_tc':>6} "
             f"{'td_tc':>6} {'VALU/w':>7} {'VMEM/w':>6}"]
    for tag, shape, c in res:
        d = derived(c)
        k = c.get("_kernel", "?")
        k = k.split("::")[-1].split("(")[0] if "::" in k else k
        lines.append(f"{tag + ' ' + shape:<18} {k[:36]:<36} {d['occupancy']:>6.2f} "
                     f"{d['vmem_lat']:>8.0f} {d['l2_lat']:>7.0f} {d['lds_lat']:>7.1f} "
                     f"{d['lds_util']:>5.1f} {d['wait_lds']:>8.3f} {d['ta_tc']:>6.3f} "
                     f"{d['td_tc']:>6.3f} {d['valu_per_wave']:>7.1f} "
                     f"{d['vmem_per_wave']:>6.1f}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--cases", default=",".join(DEFAULT_CASES))
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--out", default=None, help="also write the report here")
    a = ap.parse_args(argv)
    from .. import _capi
    version = _capi.version()          # loads the library; no GPU call
    res = []
    with tempfile.TemporaryDirectory(prefix="cq_ctr_", dir=os.environ.get("TMPDIR", "/tmp")) as t:
        for case in a.cases.split(","):
            tag, shape = case.split(":")
            res.append((tag, shape, run_case(tag, shape, a.steps, Path(t))))
    raw = []
    for tag, shape, c in res:
        raw.append(f"--- {tag} {shape} ({c.get('_kernel', '?')[:90]})")
        for k in sorted(x for x in c if not x.startswith("_")):
            raw.append(f"  {k:<30} {c[k]:>16.2f}")
    report = (f"library: {version}\n" + table(res) + "\n\nraw per-dispatch medians:\n"
              + "\n".join(raw))
    print(report)
    if a.out:
        Path(a.out).write_text(report + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
