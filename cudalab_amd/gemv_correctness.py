"""FP16/FP32 GEMV correctness suite (per variant).

Drop-in for `cudalab/gemv_correctness.py:108-311`.

Gate.  For each output row n let a_k = W[n,k] * x[k] (stored values,
promoted exactly), exact = sum_k a_k and S_n = sum_k |a_k| (fp64).  Every
FP32 accumulation of the K products in any order, each product and each
addition rounded at most once, satisfies
    |y - exact| <= 2*K*2^-24*S_n + 1/2 ulp_dtype(|y|),
and the suite gates on TOL_K = 2 times that bound, covering the binade of
both y and exact:
    tol = 2 * (2*K*2^-24*S_n + 1/2 ulp(|y|) + 1/2 ulp(|exact|))
    arith_ratio = max_n |y - exact| / tol <= 1,  y and ref finite.
The reference formulation gemv_ref (FP32 torch.mv, cast) and the allclose
metrics are reported, never gated.

Matrix: float16 and float32 x (5 bench shapes + 5 edge shapes) x 5 input
modes = 100 cases; W seed 0, x seed 1 (independent streams).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass
from pathlib import Path

import torch

from .evaluator.correctness import (REL_EPS_GUARD, TOLERANCES,
                                    compute_metrics, save_suite,
                                    summarize_results)
from .evaluator.gpu import now_iso
from .operators.gemv import BENCH_MATRIX_GEMV, gemv_ref, make_w, make_x

DTYPES = ("float16", "float32")
EDGE_SHAPES = [(1, 1), (1, 4096), (4096, 1), (16, 13), (8, 7)]
SHAPES = list(BENCH_MATRIX_GEMV) + EDGE_SHAPES
INPUT_MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
LARGE_SCALE = 10.0
SEED = 0

TOL_K = 2.0
_PER_TERM_ROUNDINGS = 2.0
_NEG24 = 2.0 ** -24


def _ulp(v: torch.Tensor, dtype_name: str) -> torch.Tensor:
    """Spacing of the target dtype's grid at |v| (ulp(0) = smallest
    subnormal)."""
    if dtype_name == "float32":
        vf = v.float().abs()
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
    atol: float
    rtol: float
    note: str = ""


def arith_ratio(y: torch.Tensor, W: torch.Tensor, x: torch.Tensor,
                dtype_name: str) -> tuple[float, float, float]:
    """(max ratio, max tol, max S) of the fixed bound; non-finite elements
    get ratio 0 (the finiteness gate judges them)."""
    if W.numel() == 0:
        return 0.0, 0.0, 0.0
    K = W.size(1)
    wd, xd = W.double(), x.double()
    S = (wd.abs() * xd.abs().unsqueeze(0)).sum(dim=1)
    exact = torch.mv(wd, xd)
    tol = TOL_K * (_PER_TERM_ROUNDINGS * K * _NEG24 * S
                   + 0.5 * _ulp(y, dtype_name).double()
                   + 0.5 * _ulp(exact, dtype_name).double())
    diff = (y.double() - exact).abs()
    ratio = torch.where(diff.isfinite() & tol.isfinite(), diff / tol,
                        torch.zeros_like(diff))
    return float(ratio.max()), float(tol.max()), float(S.max())


def check_one(variant: str, ext, W: torch.Tensor, x: torch.Tensor,
              mode: str, seed: int = SEED, note: str = "") -> CheckResult:
    y = ext.forward(variant, W, x).contiguous()
    ref = gemv_ref(W, x)
    dtype_name = str(W.dtype).split(".")[-1]
    ratio, tol_max, S_max = arith_ratio(y, W, x, dtype_name)
    ref_nan = bool(torch.isnan(ref).any())
    ref_inf = bool(torch.isinf(ref).any())
    if ref_nan or ref_inf:
        note = (note + "; reference not finite (suite construction error)"
                ).strip("; ")
    m = compute_metrics(y, ref, dtype_name)
    N, K = W.shape
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
        atol=m["atol"], rtol=m["rtol"], note=note)


def run_suite(variant: str, ext, dtypes: tuple = DTYPES,
              shapes: tuple = tuple(SHAPES),
              modes: tuple = INPUT_MODES) -> list[CheckResult]:
    """The 100-case suite of one variant (deterministic)."""
    results = []
    for dtype_name in dtypes:
        dtype = getattr(torch, dtype_name)
        for (N, K) in shapes:
            for mode in modes:
                W = make_w(N, K, dtype, seed=SEED, mode=mode, large=LARGE_SCALE)
                x = make_x(K, dtype, seed=SEED + 1, mode=mode, large=LARGE_SCALE)
                results.append(check_one(variant, ext, W, x, mode, seed=SEED))
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
        "operator": "gemv",
        "suite": "gemv-correctness",
        "generated": now_iso(),
        "gate": "pass = y and ref finite AND arith_max_ratio <= 1 (fixed "
                "bound TOL_K*(2*K*2^-24*S + ulp/2 terms on the dtype grid) "
                "against the exact fp64 GEMV)",
        "reference": "gemv_ref: fp16 -> torch.mv(W.float(), x.float()) cast "
                     "to fp16; fp32 -> torch.mv(W, x); exact = fp64 W @ x",
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
