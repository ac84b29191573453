"""INT8 per-row quantizer contract on CPU (cudalab/qgemv_quantize.py:33-119
of the reference), checked in closed form and against the CPU oracle."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cudalab_amd.qgemv_quantize import (INT8_MAX, dequantize_w,
                                        fidelity_metrics, quantize_w)
from oracle import oracle as orc


def test_quantizer_closed_form():
    torch.manual_seed(2)
    W = (torch.randn(6, 300) * 0.02).to(torch.float16)
    W[4] = 0
    Wq, s = quantize_w(W)
    assert Wq.dtype == torch.int8 and s.dtype == torch.float32
    assert tuple(s.shape) == (6,)
    Wf = W.float()
    amax = Wf.abs().amax(dim=1)
    assert torch.equal(s, amax / 127)
    safe = torch.where(s == 0, torch.ones_like(s), s)
    q_ref = torch.round(Wf / safe.unsqueeze(1)).clamp(-127, 127)
    q_ref[4] = 0
    assert torch.equal(Wq.to(torch.float32), q_ref)
    assert int(Wq.abs().max()) <= INT8_MAX
    assert float(s[4]) == 0.0 and bool((Wq[4] == 0).all())
    nz = s > 0
    err = (Wf - Wq.float() * s.unsqueeze(1)).abs()
    assert bool((err[nz] <= 0.5 * s[nz].unsqueeze(1) * (1 + 1e-5)).all())


def test_quantizer_matches_oracle():
    rng = np.random.default_rng(41)
    for scale in (0.02, 1.0, 1e-4, 10.0):
        W = (rng.standard_normal((7, 129)) * scale).astype(np.float16)
        Wq, s = quantize_w(torch.from_numpy(W))
        wq_n, s_n = orc.quantize_w8(W)
        wq_c, s_c = orc.quantize_w8_c(W)
        assert np.array_equal(Wq.numpy(), wq_n) and np.array_equal(Wq.numpy(), wq_c)
        assert np.array_equal(s.numpy(), s_n) and np.array_equal(s.numpy(), s_c)


@pytest.mark.parametrize("make", [
    lambda: quantize_w(torch.randn(4, dtype=torch.float16)),
    lambda: quantize_w(torch.randn(2, 4)),
    lambda: quantize_w(torch.randn(4, 2, dtype=torch.float16).t()),
    lambda: quantize_w(torch.tensor([[1.0, float("nan")]], dtype=torch.float16)),
    lambda: quantize_w(torch.tensor([[1.0, float("inf")]], dtype=torch.float16)),
])
def test_rejections(make):
    with pytest.raises(ValueError):
        make()


def test_dequantize_and_fidelity():
    torch.manual_seed(3)
    W = torch.randn(4, 64, dtype=torch.float16)
    x = torch.randn(64, dtype=torch.float16)
    Wq, s = quantize_w(W)
    Wd = dequantize_w(Wq, s)
    assert torch.equal(Wd, Wq.float() * s.unsqueeze(1))
    fid = fidelity_metrics(W, x, Wq, s)
    assert math.isfinite(fid["max_abs"]) and fid["cosine"] > 0.99
    assert fid["max_dequant_step_err"] <= 0.5 + 1e-4
    assert fidelity_metrics(W, torch.zeros(64, dtype=torch.float16), Wq, s)["cosine"] is None
