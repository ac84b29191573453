"""Timestamps and best-effort GPU state snapshots.

Role of `cudalab/evaluator/gpu.py` (nvidia-smi snapshots), with amd-smi /
rocm-smi on MI355X.  Never raises: a missing tool yields {"available":
False}."""
from __future__ import annotations

import datetime as _dt
import json
import shutil
import subprocess


def now_iso() -> str:
    return _dt.datetime.now(_dt.timezone.utc).astimezone().isoformat(
        timespec="seconds")


def gpu_state(device_index: int = 0, timeout: float = 10.0) -> dict:
    """Clock/temperature/power snapshot of one GPU via amd-smi (JSON)."""
    tool = shutil.which("amd-smi")
    if tool is None:
        return {"available": False, "reason": "amd-smi not found"}
    try:
        r = subprocess.run([tool, "metric", "-g", str(device_index), "-c",
                            "-t", "-p", "--json"], capture_output=True,
                           text=True, timeout=timeout)
        if r.returncode != 0:
            return {"available": False, "reason": r.stderr.strip()[:200]}
        return {"available": True, "amd_smi": json.loads(r.stdout)}
    except Exception as e:  # noqa: BLE001
        return {"available": False, "reason": f"{type(e).__name__}: {e}"[:200]}
