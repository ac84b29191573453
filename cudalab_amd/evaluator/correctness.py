"""Shared correctness metrics (report-only closeness; the GEMV gate is the
fixed accumulation-error bound of each operator's suite).

Drop-in for `cudalab/evaluator/correctness.py:27-90`: the same TOLERANCES
table, REL_EPS_GUARD, compute_metrics, summarize_results and save_suite.
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Callable, Optional

import torch

# Fixed allclose tolerances, identical for every variant (reported only).
TOLERANCES = {
    "float16": {"atol": 2e-3, "rtol": 5e-3},
    "float32": {"atol": 1e-5, "rtol": 1e-4},
}
# Denominator guard of the relative error near zero.
REL_EPS_GUARD = 1e-3


def compute_metrics(y: torch.Tensor, ref: torch.Tensor, dtype_name: str,
                    rel_eps_guard: float = REL_EPS_GUARD,
                    extra: Optional[Callable[[torch.Tensor, torch.Tensor], dict]]
                    = None) -> dict:
    """max_abs / max_rel / NaN / Inf / allclose of y against ref."""
    tol = TOLERANCES[dtype_name]
    yf, rf = y.float(), ref.float()
    diff = (yf - rf).abs()
    empty = y.numel() == 0
    m = {
        "max_abs_error": 0.0 if empty else round(float(diff.max()), 12),
        "max_rel_error": 0.0 if empty else round(
            float((diff / rf.abs().clamp_min(rel_eps_guard)).max()), 12),
        "has_nan": bool(torch.isnan(y).any()),
        "has_inf": bool(torch.isinf(y).any()),
        "ok_close": bool(torch.allclose(yf, rf, atol=tol["atol"],
                                        rtol=tol["rtol"])),
        "atol": tol["atol"],
        "rtol": tol["rtol"],
    }
    if extra is not None:
        m.update(extra(y, ref))
    return m


def summarize_results(results: list[dict]) -> dict:
    """Counts and maxima over result records (each has "pass"); failed
    records are kept (first 20)."""
    failed = [r for r in results if not r["pass"]]
    return {
        "n_total": len(results),
        "n_pass": len(results) - len(failed),
        "n_fail": len(failed),
        "all_pass": not failed,
        "max_abs_error": max((r["max_abs_error"] for r in results), default=0.0),
        "max_rel_error": max((r["max_rel_error"] for r in results), default=0.0),
        "failed": failed[:20],
    }


def save_suite(path: Path, doc: dict) -> Path:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
    return path
