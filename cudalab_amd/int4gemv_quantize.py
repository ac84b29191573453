"""W4A16 group-wise INT4 quantization contract (symmetric, zero point 0).

Drop-in for `cudalab/int4gemv_quantize.py:41-197`: same names, arguments,
results and ValueError rejections.

Contract (the operator's data format):
    W_packed  uint8 (N, K/2)  two INT4 per byte
    scale     fp16  (N, K/128), group size G = 128
    q in [-7, 7], zero point 0
    scale32[n,g] = max|W[n, g*128:(g+1)*128]| / 7     (computed in FP32)
    q[n,k]       = clamp(round_half_even(W[n,k] / scale32), -7, 7)
    an all-zero group has scale 0 and q = 0 (no division by zero, no NaN)
    scale is *stored* as fp16(scale32): kernels and references read the
    stored fp16 value.
Nibble packing: byte b of a row holds element 2b in bits 0-3 and element
2b+1 in bits 4-7, each as 4-bit two's complement (v & 0xF); unpacking
sign-extends (codes 8..15 are -8..-1).

Quantization and packing run offline, outside every timed region.  The
functions work on CPU and GPU tensors alike: `quantize_w` of a CUDA tensor
runs the on-device HIP quantizer (one launch, bit-identical to the torch
formulation `quantize_w_torch`, which serves CPU tensors).
"""
from __future__ import annotations

import torch

INT4_MAX = 7
GROUP_SIZE = 128


def _check_w(W: torch.Tensor, finite: bool = True) -> None:
    if W.dim() != 2:
        raise ValueError(f"expected a 2-D W (N, K), got {W.dim()}-D")
    if W.dtype != torch.float16:
        raise ValueError(f"the quantizer takes fp16 weights only, got {W.dtype}")
    if not W.is_contiguous():
        raise ValueError("the quantizer requires a contiguous W")
    if W.size(1) % GROUP_SIZE != 0:
        raise ValueError(f"K must be divisible by {GROUP_SIZE} "
                         f"(group size), got K={W.size(1)}")
    if finite and not bool(torch.isfinite(W).all()):
        raise ValueError(_NONFINITE)


_NONFINITE = "the quantizer requires finite W (NaN/Inf found)"


def _scale32(amax: torch.Tensor, qmax: int, rcp: bool | None) -> torch.Tensor:
    """amax / qmax in FP32: as written (torch's own per-device rounding) for
    rcp None, else forced to amax * fl(1/qmax) (True) or a correctly rounded
    division (False)."""
    if rcp is None:
        return amax / qmax
    if rcp:
        # fl32(1/qmax), held exactly by a Python float; the product rounds once
        inv = (torch.ones((), dtype=torch.float32) / qmax).item()
        return amax * inv
    # a divisor tensor on amax's own device: a true division everywhere
    return amax / torch.tensor(float(qmax), dtype=torch.float32, device=amax.device)


def quantize_w(W: torch.Tensor, semantics: str | None = None
               ) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric group-wise INT4 quantization of fp16 W (N, K), K % 128 == 0.

    Returns (W_packed uint8 (N, K/2), scale fp16 (N, K/128)).
    Raises ValueError for non-2-D, non-fp16, non-contiguous, K % 128 != 0,
    or non-finite input.

    A CUDA W is quantized and packed by the HIP kernel (cq_int4_quantize)
    in one pass; its non-finite check reads the scale, which is non-finite
    exactly where a group of W holds NaN/Inf.  An empty W launches nothing
    and gets the torch formulation's empty results.

    `semantics` picks how `amax / qmax` is rounded, as the reference's
    torch code does on each device: "cpu" one correctly rounded division,
    "gpu" amax * fl(1/qmax) (torch applies a CPU-scalar divisor on a GPU as
    its reciprocal).  The default is W's own device, so the result equals
    the reference's `quantize_w` on the same tensor."""
    if semantics not in (None, "cpu", "gpu"):
        raise ValueError(f"semantics must be None, 'cpu' or 'gpu', got {semantics!r}")
    if W.is_cuda and W.numel() > 0:
        _check_w(W, finite=False)
        from .ext import quantize_int4
        W_packed, scale = quantize_int4(W, rcp=semantics != "cpu")
        if not bool(torch.isfinite(scale).all()):
            raise ValueError(_NONFINITE)
        return W_packed, scale
    return quantize_w_torch(W, rcp=None if semantics is None else semantics == "gpu")


def quantize_w_torch(W: torch.Tensor, rcp: bool | None = None
                     ) -> tuple[torch.Tensor, torch.Tensor]:
    """The quantizer as torch tensor operations (the reference's
    formulation, cudalab/int4gemv_quantize.py:61-89), on W's device.
    `rcp` None divides by the Python number as the reference does (torch
    rounds that per device); True / False force amax * fl(1/7) / amax / 7."""
    _check_w(W)
    N, K = W.shape
    G = K // GROUP_SIZE
    groups = W.float().reshape(N, G, GROUP_SIZE)
    s32 = _scale32(groups.abs().amax(dim=2), INT4_MAX, rcp)   # (N, G) FP32
    is_zero = s32 == 0
    denom = torch.where(is_zero, torch.ones_like(s32), s32)
    q = torch.round(groups / denom.unsqueeze(2))        # half to even
    q = q.clamp(-INT4_MAX, INT4_MAX)
    q = q.masked_fill(is_zero.unsqueeze(2), 0.0)
    W_packed = pack_q(q.reshape(N, K).to(torch.int32))
    return W_packed, s32.to(torch.float16).contiguous()


def pack_q(q: torch.Tensor) -> torch.Tensor:
    """INT4 values (N, K) int32/int64 in [-8, 7], K even -> uint8 (N, K/2).

    Element 2b goes to the low nibble of byte b, element 2b+1 to the high
    nibble, each as v & 0xF."""
    if q.dim() != 2:
        raise ValueError(f"pack_q expects a 2-D (N, K) tensor, got {q.dim()}-D")
    N, K = q.shape
    if K % 2 != 0:
        raise ValueError(f"pack_q needs an even K, got K={K}")
    if q.numel() and (int(q.min()) < -8 or int(q.max()) > 7):
        raise ValueError("pack_q: values outside the INT4 two's complement "
                         "range [-8, 7]")
    pairs = q.to(torch.int32).reshape(N, K // 2, 2) & 0xF
    return (pairs[..., 0] | (pairs[..., 1] << 4)).to(torch.uint8).contiguous()


def unpack_w(W_packed: torch.Tensor) -> torch.Tensor:
    """uint8 (N, K/2) -> int32 (N, K) in [-8, 7]; exact inverse of pack_q."""
    if W_packed.dim() != 2:
        raise ValueError(f"unpack_w expects a 2-D (N, K/2) tensor, got "
                         f"{W_packed.dim()}-D")
    if W_packed.dtype != torch.uint8:
        raise ValueError(f"unpack_w takes uint8 only, got {W_packed.dtype}")
    N, H = W_packed.shape
    b = W_packed.to(torch.int32)
    nib = torch.stack((b & 0xF, b >> 4), dim=-1)         # (N, H, 2)
    vals = nib - ((nib & 0x8) << 1)                      # sign-extend 4 bits
    return vals.reshape(N, 2 * H).contiguous()


def dequantize_w(W_packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """FP32 W_dequant[n,k] = q[n,k] * float(scale[n, k/128]) (stored fp16
    scale promoted; the product is exact in FP32)."""
    q = unpack_w(W_packed)
    N, K = q.shape
    if tuple(scale.shape) != (N, K // GROUP_SIZE):
        raise ValueError(f"scale shape {tuple(scale.shape)} does not match "
                         f"({N}, {K // GROUP_SIZE})")
    s = scale.float().repeat_interleave(GROUP_SIZE, dim=1)
    return q.float() * s


def fidelity_metrics(W: torch.Tensor, x: torch.Tensor,
                     W_packed: torch.Tensor, scale: torch.Tensor) -> dict:
    """Quantization fidelity (report-only): y_orig = W @ x vs
    y_quant = W_dequant @ x, both FP32; cosine is None for a zero vector.
    Also the quantizer self-checks max |W - q*s16| and max |W - q*s16| / s
    (denominator clamped at 1e-30)."""
    xf = x.float()
    y_orig = torch.mv(W.float(), xf)
    Wd = dequantize_w(W_packed, scale)
    y_quant = torch.mv(Wd, xf)
    diff = y_quant - y_orig
    n_o = float(y_orig.norm())
    n_q = float(y_quant.norm())
    cosine = (float(torch.dot(y_orig, y_quant)) / (n_o * n_q)
              if n_o > 0 and n_q > 0 else None)
    s = scale.float().clamp_min(1e-30).repeat_interleave(GROUP_SIZE, dim=1)
    deq = (W.float() - Wd).abs()
    q = unpack_w(W_packed)
    return {
        "max_abs": float(diff.abs().max()) if diff.numel() else 0.0,
        "rmse": float(diff.pow(2).mean().sqrt()) if diff.numel() else 0.0,
        "cosine": cosine,
        "y_orig_norm": n_o,
        "y_quant_norm": n_q,
        "max_dequant_abs_err": float(deq.max()) if deq.numel() else 0.0,
        "max_dequant_step_err": float((deq / s).max()) if deq.numel() else 0.0,
        "n_zero_scale_groups": int((scale == 0).sum()),
        "max_abs_q": int(q.abs().max()) if q.numel() else 0,
        "note": "quantization fidelity: quantization error, not a kernel "
                "bug; reported only, never a kernel-correctness gate",
    }
