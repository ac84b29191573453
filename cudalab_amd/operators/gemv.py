"""Seeded fp16 input generators shared by the quantized GEMV operators.

Drop-in for `make_w` / `make_x` of `cudalab/operators/gemv.py:106-190`
(same modes and arguments).  Difference by design: the random stream comes
from a CPU `torch.Generator` and the tensor is then moved to `device`, so
the same seed gives the same values on every host (the reference drew on
the GPU generator, whose stream is tied to the device).

Modes:
  normal      N(0, scale)
  zeros       all zero
  tiny        N(0, 1e-4)   (many fp16 subnormals in x)
  large       N(0, large)
  mixed_sign  W: |N(0,1)| * (-1)^(i+j);  x: |N(0,1)| * independent random
              signs, so that W[i,j]*x[j] has independent signs along a row
              (real cancellation).
"""
from __future__ import annotations

import torch

MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    return g


def make_w(N: int, K: int, dtype: torch.dtype, device: str = "cuda",
           seed: int = 0, mode: str = "normal", scale: float = 1.0,
           large: float = 10.0) -> torch.Tensor:
    g = _gen(seed)
    if mode == "normal":
        w = torch.randn(N, K, generator=g) * scale
    elif mode == "zeros":
        w = torch.zeros(N, K)
    elif mode == "tiny":
        w = torch.randn(N, K, generator=g) * 1e-4
    elif mode == "large":
        w = torch.randn(N, K, generator=g) * large
    elif mode == "mixed_sign":
        mag = torch.randn(N, K, generator=g).abs()
        parity = (torch.arange(N).unsqueeze(1) + torch.arange(K).unsqueeze(0)) % 2
        w = torch.where(parity == 0, mag, -mag)
    else:
        raise ValueError(f"unknown input mode: {mode!r}")
    return w.to(dtype).contiguous().to(device)


def make_x(K: int, dtype: torch.dtype, device: str = "cuda", seed: int = 0,
           mode: str = "normal", scale: float = 1.0,
           large: float = 10.0) -> torch.Tensor:
    g = _gen(seed)
    if mode == "normal":
        x = torch.randn(K, generator=g) * scale
    elif mode == "zeros":
        x = torch.zeros(K)
    elif mode == "tiny":
        x = torch.randn(K, generator=g) * 1e-4
    elif mode == "large":
        x = torch.randn(K, generator=g) * large
    elif mode == "mixed_sign":
        mag = torch.randn(K, generator=g).abs()
        bits = torch.randint(0, 2, (K,), generator=g)
        x = torch.where(bits == 0, mag, -mag)
    else:
        raise ValueError(f"unknown input mode: {mode!r}")
    return x.to(dtype).contiguous().to(device)
