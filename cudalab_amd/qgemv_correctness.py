"""INT8 W8A16 GEMV correctness suite (per variant).

Drop-in for `cudalab/qgemv_correctness.py:90-371`: the same fixed bound as
the INT4 suite with a_k = W_q[n,k]*scale[n]*x[k] (fp32 scale), 5 bench
shapes + 5 edge shapes (odd K included) x 5 modes = 50 cases.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Optional

import torch

from .evaluator.correctness import (REL_EPS_GUARD, TOLERANCES,
                                    compute_metrics, save_suite,
                                    summarize_results)
from .evaluator.gpu import now_iso
from .int4gemv_correctness import _ulp
from .operators.qgemv import BENCH_MATRIX_QGEMV, make_w_q, make_x_q
from .qgemv_quantize import fidelity_metrics

DTYPES = ("float16",)
EDGE_SHAPES = [(1, 1), (1, 4096), (4096, 1), (16, 13), (8, 7)]
SHAPES = list(BENCH_MATRIX_QGEMV) + EDGE_SHAPES
INPUT_MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
LARGE_SCALE = 10.0
SEED = 0

TOL_K = 2.0
_PER_TERM_ROUNDINGS = 3.0
_NEG24 = 2.0 ** -24


@dataclass
class CheckResult:
    variant: str
    shape: list
    dtype: str
    seed: int
    mode: str
    passed: bool
    arith_max_ratio: float
    has_nan: bool
    has_inf: bool
    ref_has_nan: bool
    ref_has_inf: bool
    max_abs_error: float
    max_rel_error: float
    ok_close: bool
    arith_tol_max: float
    S_max: float
    fid_max_abs: Optional[float]
    fid_max_rel: Optional[float]
    fid_rmse: Optional[float]
    fid_cosine: Optional[float]
    atol: float
    rtol: float
    note: str = ""


def arith_ratio(y: torch.Tensor, W_q: torch.Tensor, scale: torch.Tensor,
                x: torch.Tensor, dtype_name: str) -> tuple[float, float, float]:
    if W_q.numel() == 0:
        return 0.0, 0.0, 0.0
    K = W_q.size(1)
    Wd = W_q.double() * scale.double().unsqueeze(1)
    xd = x.double()
    S = (Wd.abs() * xd.abs().unsqueeze(0)).sum(dim=1)
    exact = torch.mv(Wd, xd)
    tol = TOL_K * (_PER_TERM_ROUNDINGS * K * _NEG24 * S
                   + 0.5 * _ulp(y, dtype_name).double()
                   + 0.5 * _ulp(exact, dtype_name).double())
    diff = (y.double() - exact).abs()
    ratio = torch.where(diff.isfinite() & tol.isfinite(), diff / tol,
                        torch.zeros_like(diff))
    return float(ratio.max()), float(tol.max()), float(S.max())


def check_one(variant: str, ext, W_q: torch.Tensor, scale: torch.Tensor,
              W_fp16: torch.Tensor, x: torch.Tensor, mode: str,
              seed: int = SEED, note: str = "") -> CheckResult:
    y = ext.forward(variant, W_q, scale, x).contiguous()
    ref = torch.mv(W_q.float() * scale.unsqueeze(1),
                   x.float()).to(torch.float16)
    dtype_name = str(y.dtype).split(".")[-1]
    ratio, tol_max, S_max = arith_ratio(y, W_q, scale, x, dtype_name)
    ref_nan = bool(torch.isnan(ref).any())
    ref_inf = bool(torch.isinf(ref).any())
    if ref_nan or ref_inf:
        note = (note + "; reference not finite (suite construction error)"
                ).strip("; ")
    m = compute_metrics(y, ref, dtype_name)
    fid = fidelity_metrics(W_fp16, x, W_q, scale)
    N, K = W_q.shape
    return CheckResult(
        variant=variant, shape=[int(N), int(K)], dtype=dtype_name, seed=seed,
        mode=mode,
        passed=(ratio <= 1.0 and not m["has_nan"] and not m["has_inf"]
                and not ref_nan and not ref_inf),
        arith_max_ratio=round(ratio, 12),
        has_nan=m["has_nan"], has_inf=m["has_inf"],
        ref_has_nan=ref_nan, ref_has_inf=ref_inf,
        max_abs_error=m["max_abs_error"], max_rel_error=m["max_rel_error"],
        ok_close=m["ok_close"],
        arith_tol_max=round(tol_max, 12), S_max=round(S_max, 12),
        fid_max_abs=round(fid["max_abs"], 12),
        fid_max_rel=round(fid["max_rel"], 12),
        fid_rmse=round(fid["rmse"], 12),
        fid_cosine=(round(fid["cosine"], 9) if fid["cosine"] is not None
                    else None),
        atol=m["atol"], rtol=m["rtol"], note=note)


def run_suite(variant: str, ext, dtypes: tuple = DTYPES,
              shapes: tuple = tuple(SHAPES),
              modes: tuple = INPUT_MODES) -> list[CheckResult]:
    results = []
    for _dtype in dtypes:
        for (N, K) in shapes:
            for mode in modes:
                W_q, scale, W = make_w_q(N, K, seed=SEED, mode=mode,
                                         large=LARGE_SCALE)
                x = make_x_q(K, seed=SEED + 1, mode=mode, large=LARGE_SCALE)
                results.append(check_one(variant, ext, W_q, scale, W, x, mode,
                                         seed=SEED))
    return results


def _jsonable(r: CheckResult) -> dict:
    d = asdict(r)
    d["pass"] = d.pop("passed")
    return d


def summarize(results: list[CheckResult]) -> dict:
    s = summarize_results([_jsonable(r) for r in results])
    s["max_arith_max_ratio"] = max((r.arith_max_ratio for r in results),
                                   default=0.0)
    s["ok_close_vs_ref_all"] = all(r.ok_close for r in results)
    return s


def save_results(results: list[CheckResult], out_path: Path) -> Path:
    return save_suite(out_path, {
        "operator": "qgemv",
        "suite": "qgemv-correctness",
        "generated": now_iso(),
        "gate": "pass = y and ref finite AND arith_max_ratio <= 1",
        "matrix": {"dtypes": list(DTYPES),
                   "shapes_NxK": [list(s) for s in SHAPES],
                   "input_modes": list(INPUT_MODES),
                   "seed_w": SEED, "seed_x": SEED + 1},
        "tolerances_reported": TOLERANCES,
        "tol_k": TOL_K,
        "per_term_roundings": _PER_TERM_ROUNDINGS,
        "rel_eps_guard": REL_EPS_GUARD,
        "summary": summarize(results),
        "results": [_jsonable(r) for r in results],
    })


FIDELITY_SHAPES = list(BENCH_MATRIX_QGEMV)


def run_fidelity_suite(seed: int = SEED) -> dict:
    cases = []
    for (N, K) in FIDELITY_SHAPES:
        for mode in INPUT_MODES:
            W_q, scale, W = make_w_q(N, K, seed=seed, mode=mode,
                                     large=LARGE_SCALE)
            x = make_x_q(K, seed=seed + 1, mode=mode, large=LARGE_SCALE)
            cases.append({"shape": [int(N), int(K)], "mode": mode,
                          **fidelity_metrics(W, x, W_q, scale)})
    cosines = [c["cosine"] for c in cases if c["cosine"] is not None]
    return {
        "seed_w": seed, "seed_x": seed + 1,
        "summary": {
            "n_cases": len(cases),
            "max_fid_max_abs": max(c["max_abs"] for c in cases),
            "max_fid_rmse": max(c["rmse"] for c in cases),
            "min_cosine": min(cosines) if cosines else None,
            "max_dequant_step_err": max(c["max_dequant_step_err"]
                                        for c in cases),
            "max_abs_q": max(c["max_abs_q"] for c in cases),
        },
        "cases": cases,
    }


def save_fidelity(fid: dict, out_path: Path) -> Path:
    out_path = Path(out_path)
    out_path.parent.mkdir(parents=True, exist_ok=True)
    doc = {"operator": "qgemv", "suite": "qgemv-quantization-fidelity",
           "generated": now_iso(), **fid}
    out_path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
    return out_path
