"""Registers, LDS and occupancy limits of the kernel instances the library
plans for a set of shapes (no GPU needed).

Usage: python -m cudalab_amd.evaluator.resources [--json FILE]

Compiles csrc/cq_kernels.hip for gfx950 with the library's own flags and
the compiler's resource-usage remarks (-Rpass-analysis=kernel-resource-usage),
asks the library which kernel instance and launch shape each (operator,
shape) runs (cq_describe_launch: kernel, rows per lane, workgroup size, grid
and dynamic LDS bytes per workgroup), and reports per instance:

  VGPRs, AGPRs, SGPRs, scratch bytes per lane, and the compiler's waves per
  SIMD (the register limit, launch bounds included);
  the LDS limit: workgroups per CU that fit 160 KiB of LDS, in waves per
  SIMD;
  the occupancy limit, the smaller of the two (at most 8 waves per SIMD);
  the grid's waves per SIMD if every workgroup were resident at once
  (grid x waves per workgroup / 1024 SIMDs).

The measured mean occupancy of the same launches (rocprofv3's
MeanOccupancyPerCU) is in profiles/, next to this table.
"""
from __future__ import annotations

import argparse
import json
import re
import subprocess
import sys
import tempfile
from pathlib import Path

from .. import _capi
from ..build import CSRC, HIPCC_FLAGS, INCLUDE, hipcc

LDS_PER_CU = 160 * 1024
SIMDS = 1024                 # 256 CUs x 4 SIMDs
MAX_WAVES_PER_SIMD = 8

CASES = (("int4gemv", "int4gemv_cdna4", 1024, 4096),
         ("int4gemv", "int4gemv_cdna4", 4096, 1024),
         ("int4gemv", "int4gemv_cdna4", 4096, 4096),
         ("int4gemv", "int4gemv_cdna4", 11008, 4096),
         ("int4gemv", "int4gemv_cdna4", 4096, 11008),
         ("int4gemv", "int4gemv_cdna4", 8192, 8192),
         ("int4gemv", "int4gemv_cdna4", 4096, 28672),
         ("int4gemv", "int4gemv_cdna4", 8192, 28672),
         ("qgemv", "qgemv_cdna4", 1024, 4096),
         ("qgemv", "qgemv_cdna4", 4096, 1024),
         ("qgemv", "qgemv_cdna4", 4096, 4096),
         ("qgemv", "qgemv_cdna4", 11008, 4096),
         ("qgemv", "qgemv_cdna4", 4096, 11008),
         ("qgemv", "qgemv_cdna4", 8192, 8192),
         ("qgemv", "qgemv_cdna4", 4096, 28672),
         ("qgemv", "qgemv_cdna4", 8192, 28672))


def compile_remarks() -> dict[str, dict]:
    """Demangled kernel name -> its resource-usage figures."""
    with tempfile.TemporaryDirectory(prefix="cq_res_") as tmp:
        cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
               "--cuda-device-only", "-c", str(CSRC / "cq_kernels.hip"),
               "-o", str(Path(tmp) / "k.o"),
               "-Rpass-analysis=kernel-resource-usage"]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                           text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed ({r.returncode}):\n{r.stdout[-2000:]}")
    blocks: dict[str, dict] = {}
    cur = None
    for line in r.stdout.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = {}
            blocks[m.group(1)] = cur
            continue
        m = re.search(r"remark:\s+([A-Za-z][A-Za-z /\[\]]*?): (\d+)", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    names = list(blocks)
    dem = subprocess.run(["c++filt"], input="\n".join(names), stdout=subprocess.PIPE,
                         text=True, check=True).stdout.splitlines()
    return {d: blocks[n] for n, d in zip(names, dem)}


def instance_name(op: str, plan: dict) -> str:
    """Demangled name prefix of the kernel instance a plan launches."""
    if plan["kernel"] == "lds":
        return (f"{op}_lds_kernel<{plan['cw']}, {plan['j']}, {plan['r']}, "
                f"{plan['block']}>")
    if plan["kernel"] == "tiled":
        return f"{op}_tiled_kernel<{plan['block']}, {plan['tile']}, {plan['r']}>"
    raise ValueError(f"no instance name for plan {plan}")


def find(remarks: dict[str, dict], prefix: str) -> tuple[str, dict]:
    hits = [k for k in remarks if f"::{prefix}(" in k]
    if len(hits) != 1:
        raise KeyError(f"{prefix}: {len(hits)} matches")
    return hits[0], remarks[hits[0]]


def rows(remarks: dict[str, dict], cases=CASES) -> list[dict]:
    out = []
    for op, variant, n, k in cases:
        plan = _capi.describe_launch(op, variant, n, k, 4096, 8192)
        inst = instance_name(op, plan)
        _, rem = find(remarks, inst)
        block, grid, lds = int(plan["block"]), int(plan["grid"]), int(plan["lds"])
        waves_wg = block // 64
        reg_limit = rem.get("Occupancy [waves/SIMD]", 0)
        wg_per_cu = LDS_PER_CU // lds if lds > 0 else 10 ** 9
        lds_limit = wg_per_cu * waves_wg / 4.0
        out.append({"op": op, "variant": variant, "N": n, "K": k,
                    "kernel": inst, "block": block, "grid": grid,
                    "vgprs": rem.get("VGPRs"), "agprs": rem.get("AGPRs"),
                    "sgprs": rem.get("TotalSGPRs"),
                    "scratch": rem.get("ScratchSize [bytes/lane]"),
                    "lds_bytes": lds, "waves_per_simd_registers": reg_limit,
                    "waves_per_simd_lds": round(min(lds_limit, MAX_WAVES_PER_SIMD), 2),
                    "waves_per_simd_limit": round(min(reg_limit, lds_limit,
                                                      MAX_WAVES_PER_SIMD), 2),
                    "grid_waves_per_simd": round(grid * waves_wg / SIMDS, 2)})
    return out


def table(rs: list[dict]) -> str:
    hdr = (f"{'op':<9} {'N':>6} {'K':>6}  {'kernel instance':<34} {'VGPR':>4} "
           f"{'AGPR':>4} {'SGPR':>4} {'scr':>3} {'LDS B':>7} {'w/SIMD reg':>10} "
           f"{'w/SIMD lds':>10} {'limit':>5} {'grid w/SIMD':>11}")
    lines = [hdr]
    for r in rs:
        lines.append(f"{r['op']:<9} {r['N']:>6} {r['K']:>6}  {r['kernel']:<34} "
                     f"{r['vgprs']:>4} {r['agprs']:>4} {r['sgprs']:>4} {r['scratch']:>3} "
                     f"{r['lds_bytes']:>7} {r['waves_per_simd_registers']:>10} "
                     f"{r['waves_per_simd_lds']:>10} {r['waves_per_simd_limit']:>5} "
                     f"{r['grid_waves_per_simd']:>11}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--json", default=None)
    a = ap.parse_args(argv)
    print(f"library: {_capi.version()}", flush=True)
    rs = rows(compile_remarks())
    print(table(rs))
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rs, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
