"""INT4 W4A16 GEMV correctness suite (per variant), layers (a) and (c).

Drop-in for `cudalab/int4gemv_correctness.py:113-420`.

(a) Kernel correctness, the gate.  For each output row n let
        a_k   = q[n,k] * s16[n,k/128] * x[k]      (stored values, exact)
        exact = sum_k a_k                          (fp64)
        S_n   = sum_k |a_k|                        (fp64)
    Every legal FP32 evaluation that rounds each term at most three times
    (q*s product, *x product or dot rounding, accumulate) and sums in any
    order satisfies
        |y - exact| <= 3*K*2^-24*S_n + 1/2 ulp16(|y|) + 1/2 ulp16(|exact|),
    and the suite gates on TOL_K = 2 times that bound:
        arith_ratio = max_n |y - exact| / tol <= 1,  y and ref finite.
    The FP32 CPU-style reference `dequantize_w @ x` (cast fp16) and the
    allclose metrics are reported, never gated.
(c) Quantization fidelity against the unquantized fp16 W, reported only.

Matrix: the 5 bench shapes + 5 edge shapes x 5 input modes = 50 cases; W
seed 0, x seed 1 (independent streams).
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
from .int4gemv_quantize import (GROUP_SIZE, dequantize_w, fidelity_metrics,
                                unpack_w)
from .operators.int4gemv import BENCH_MATRIX_INT4GEMV, make_w4, make_x4

DTYPES = ("float16",)
EDGE_SHAPES = [(1, 128), (1, 4096), (3, 128), (16, 256), (8, 128)]
SHAPES = list(BENCH_MATRIX_INT4GEMV) + EDGE_SHAPES
INPUT_MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
LARGE_SCALE = 10.0
SEED = 0

TOL_K = 2.0
_PER_TERM_ROUNDINGS = 3.0
_NEG24 = 2.0 ** -24


def _ulp(v: torch.Tensor, dtype_name: str) -> torch.Tensor:
    """Spacing of the target dtype's grid at |v| (ulp(0) = smallest
    subnormal)."""
    if dtype_name == "float32":
        vf = v.float()
        return torch.nextafter(vf, torch.full_like(vf, float("inf"))) - vf
    a = v.half().float().abs()
    tiny16 = torch.finfo(torch.float16).tiny          # 2^-14
    e = torch.floor(torch.log2(a.clamp_min(tiny16)))
    return torch.where(a >= tiny16, torch.pow(2.0, e - 10),
                       torch.full_like(a, 2.0 ** -24))


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
    fid_rmse: Optional[float]
    fid_cosine: Optional[float]
    atol: float
    rtol: float
    note: str = ""


def arith_ratio(y: torch.Tensor, W_packed: torch.Tensor,
                scale: torch.Tensor, x: torch.Tensor,
                dtype_name: str) -> tuple[float, float, float]:
    """(max ratio, max tol, max S) of the fixed bound; non-finite elements
    get ratio 0 (the finiteness gate judges them)."""
    if W_packed.numel() == 0:
        return 0.0, 0.0, 0.0
    K = 2 * W_packed.size(1)
    q = unpack_w(W_packed).double()
    s = scale.double().repeat_interleave(GROUP_SIZE, dim=1)
    xd = x.double()
    qs = q * s
    S = (qs.abs() * xd.abs().unsqueeze(0)).sum(dim=1)
    exact = torch.mv(qs, xd)
    tol = TOL_K * (_PER_TERM_ROUNDINGS * K * _NEG24 * S
                   + 0.5 * _ulp(y, dtype_name).double()
                   + 0.5 * _ulp(exact, dtype_name).double())
    diff = (y.double() - exact).abs()
    ratio = torch.where(diff.isfinite() & tol.isfinite(), diff / tol,
                        torch.zeros_like(diff))
    return float(ratio.max()), float(tol.max()), float(S.max())


def check_one(variant: str, ext, W_packed: torch.Tensor, scale: torch.Tensor,
              W_fp16: torch.Tensor, x: torch.Tensor, mode: str,
              seed: int = SEED, note: str = "") -> CheckResult:
    y = ext.forward(variant, W_packed, scale, x).contiguous()
    ref = torch.mv(dequantize_w(W_packed, scale), x.float()).to(torch.float16)
    dtype_name = str(y.dtype).split(".")[-1]
    ratio, tol_max, S_max = arith_ratio(y, W_packed, scale, x, dtype_name)
    ref_nan = bool(torch.isnan(ref).any())
    ref_inf = bool(torch.isinf(ref).any())
    if ref_nan or ref_inf:
        note = (note + "; reference not finite (suite construction error)"
                ).strip("; ")
    m = compute_metrics(y, ref, dtype_name)
    fid = fidelity_metrics(W_fp16, x, W_packed, scale)
    N, K = W_packed.size(0), 2 * W_packed.size(1)
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
        fid_max_abs=round(fid["max_abs"], 12), fid_rmse=round(fid["rmse"], 12),
        fid_cosine=(round(fid["cosine"], 9) if fid["cosine"] is not None
                    else None),
        atol=m["atol"], rtol=m["rtol"], note=note)


def run_suite(variant: str, ext, dtypes: tuple = DTYPES,
              shapes: tuple = tuple(SHAPES),
              modes: tuple = INPUT_MODES) -> list[CheckResult]:
    """The 50-case layer-(a) suite of one variant (deterministic)."""
    results = []
    for _dtype in dtypes:
        for (N, K) in shapes:
            for mode in modes:
                W_packed, scale, W = make_w4(N, K, seed=SEED, mode=mode,
                                             large=LARGE_SCALE)
                x = make_x4(K, seed=SEED + 1, mode=mode, large=LARGE_SCALE)
                results.append(check_one(variant, ext, W_packed, scale, W, x,
                                         mode, seed=SEED))
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
        "operator": "int4gemv",
        "suite": "int4gemv-correctness",
        "generated": now_iso(),
        "gate": "pass = y and ref finite AND arith_max_ratio <= 1 (fixed "
                "bound TOL_K*(3*K*2^-24*S + ulp16/2 terms) against the exact "
                "fp64 dequantized GEMV)",
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


FIDELITY_SHAPES = list(BENCH_MATRIX_INT4GEMV)


def run_fidelity_suite(seed: int = SEED) -> dict:
    """Layer (c): quantization fidelity over 5 shapes x 5 modes."""
    cases = []
    for (N, K) in FIDELITY_SHAPES:
        for mode in INPUT_MODES:
            W_packed, scale, W = make_w4(N, K, seed=seed, mode=mode,
                                         large=LARGE_SCALE)
            x = make_x4(K, seed=seed + 1, mode=mode, large=LARGE_SCALE)
            cases.append({"shape": [int(N), int(K)], "mode": mode,
                          **fidelity_metrics(W, x, W_packed, scale)})
    cosines = [c["cosine"] for c in cases if c["cosine"] is not None]
    return {
        "seed_w": seed, "seed_x": seed + 1,
        "matrix": {"shapes_NxK": [list(s) for s in FIDELITY_SHAPES],
                   "input_modes": list(INPUT_MODES)},
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
    doc = {"operator": "int4gemv", "suite": "int4gemv-quantization-fidelity",
           "generated": now_iso(), **fid}
    out_path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
    return out_path
