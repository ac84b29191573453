"""W8A16 per-row INT8 quantization contract (symmetric, zero point 0).

Drop-in for `cudalab/qgemv_quantize.py:30-119`.

    scale[n] = max_k |W[n,k]| / 127           (FP32, stored as FP32 (N,))
    q[n,k]   = clamp(round_half_even(W[n,k] / scale[n]), -127, 127)
    an all-zero row has scale 0 and q = 0.

The scale stays FP32: the reference's kernel boundary requires a 1-D
float32 scale and rejects fp16 (kernels/qgemv/bindings.cpp:76-88,
cudalab/qgemv_negative.py:145-148).
"""
from __future__ import annotations

import torch

INT8_MAX = 127


_NONFINITE = "the quantizer requires finite W (NaN/Inf found)"


def _check_w(W: torch.Tensor, finite: bool = True) -> None:
    if W.dim() != 2:
        raise ValueError(f"expected a 2-D W (N, K), got {W.dim()}-D")
    if W.dtype != torch.float16:
        raise ValueError(f"the quantizer takes fp16 weights only, got {W.dtype}")
    if not W.is_contiguous():
        raise ValueError("the quantizer requires a contiguous W")
    if finite and not bool(torch.isfinite(W).all()):
        raise ValueError(_NONFINITE)


def quantize_w(W: torch.Tensor, semantics: str | None = None
               ) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-row INT8 quantization of fp16 W (N, K).

    Returns (W_q int8 (N, K), scale float32 (N,)).  Raises ValueError for
    non-2-D, non-fp16, non-contiguous or non-finite input.

    A CUDA W is quantized by the HIP kernel (cq_q8_quantize) in one launch;
    its non-finite check reads the scale, which is non-finite exactly for
    the rows of W holding NaN/Inf.  An empty W launches nothing and gets
    the torch formulation's result.

    `semantics` picks how `amax / qmax` is rounded, as the reference's
    torch code does on each device: "cpu" one correctly rounded division,
    "gpu" amax * fl(1/qmax) (torch applies a CPU-scalar divisor on a GPU as
    its reciprocal).  The default is W's own device, so the result equals
    the reference's `quantize_w` on the same tensor."""
    if semantics not in (None, "cpu", "gpu"):
        raise ValueError(f"semantics must be None, 'cpu' or 'gpu', got {semantics!r}")
    if W.is_cuda and W.numel() > 0:
        _check_w(W, finite=False)
        from .ext import quantize_q8
        W_q, scale = quantize_q8(W, rcp=semantics != "cpu")
        if not bool(torch.isfinite(scale).all()):
            raise ValueError(_NONFINITE)
        return W_q, scale
    return quantize_w_torch(W, rcp=None if semantics is None else semantics == "gpu")


def quantize_w_torch(W: torch.Tensor, rcp: bool | None = None
                     ) -> tuple[torch.Tensor, torch.Tensor]:
    """The quantizer as torch tensor operations (the reference's
    formulation, cudalab/qgemv_quantize.py:33-64), on W's device.  `rcp` as
    in int4gemv_quantize.quantize_w_torch."""
    from .int4gemv_quantize import _scale32
    _check_w(W)
    Wf = W.float()
    scale = _scale32(Wf.abs().amax(dim=1), INT8_MAX, rcp)  # (N,) FP32
    is_zero = scale == 0
    denom = torch.where(is_zero, torch.ones_like(scale), scale)
    q = torch.round(Wf / denom.unsqueeze(1)).clamp(-INT8_MAX, INT8_MAX)
    q = q.masked_fill(is_zero.unsqueeze(1), 0.0)
    return q.to(torch.int8), scale


def dequantize_w(W_q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """FP32 W_dequant = W_q * scale[:, None]."""
    return W_q.float() * scale.unsqueeze(1)


def fidelity_metrics(W: torch.Tensor, x: torch.Tensor, W_q: torch.Tensor,
                     scale: torch.Tensor) -> dict:
    """Quantization fidelity (report-only): max_abs / max_rel / RMSE /
    cosine of y_quant vs y_orig (FP32), plus quantizer self-checks."""
    xf = x.float()
    y_orig = torch.mv(W.float(), xf)
    Wd = dequantize_w(W_q, scale)
    y_quant = torch.mv(Wd, xf)
    diff = y_quant - y_orig
    n_o = float(y_orig.norm())
    n_q = float(y_quant.norm())
    cosine = (float(torch.dot(y_orig, y_quant)) / (n_o * n_q)
              if n_o > 0 and n_q > 0 else None)
    deq = (W.float() - Wd).abs()
    sc = scale.clamp_min(1e-30).unsqueeze(1)
    return {
        "max_abs": float(diff.abs().max()) if diff.numel() else 0.0,
        "max_rel": float((diff.abs() / y_orig.abs().clamp_min(1e-3)).max())
        if diff.numel() else 0.0,
        "rmse": float(diff.pow(2).mean().sqrt()) if diff.numel() else 0.0,
        "cosine": cosine,
        "y_orig_norm": n_o,
        "y_quant_norm": n_q,
        "max_dequant_abs_err": float(deq.max()) if deq.numel() else 0.0,
        "max_dequant_step_err": float((deq / sc).max()) if deq.numel() else 0.0,
        "n_zero_scale_rows": int((scale == 0).sum()),
        "max_abs_q": int(W_q.abs().max()) if W_q.numel() else 0,
        "note": "quantization fidelity: quantization error, not a kernel "
                "bug; reported only, never a kernel-correctness gate",
    }
