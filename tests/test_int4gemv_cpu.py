"""Layer (b) of the INT4 contract on CPU: pack/unpack bijection, quantizer
formula, zero groups, rejections, fidelity sanity, dequantize semantics.

Restates the reference's 39 checks (tests/test_int4gemv_cpu.py:53-249 of
the reference) as pytest against the product quantizer
(cudalab_amd.int4gemv_quantize), and checks the product quantizer bit for
bit against the CPU oracle (numpy and C)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cudalab_amd.int4gemv_quantize import (GROUP_SIZE, INT4_MAX, dequantize_w,
                                           fidelity_metrics, pack_q,
                                           quantize_w, unpack_w)
from oracle import oracle as orc


# [1] exhaustive 256-byte bijection
def test_exhaustive_byte_bijection():
    Wp = torch.arange(256, dtype=torch.uint8).view(1, 256)
    Wq = unpack_w(Wp)
    assert tuple(Wq.shape) == (1, 512)
    assert int(Wq.min()) >= -8 and int(Wq.max()) <= 7
    lo, hi = Wq[0, 0::2], Wq[0, 1::2]
    for b in range(256):
        exp_lo = (b & 0x0F) - 16 if (b & 0x08) else (b & 0x0F)
        exp_hi = ((b >> 4) & 0x0F) - 16 if (b & 0x80) else ((b >> 4) & 0x0F)
        assert (int(lo[b]), int(hi[b])) == (exp_lo, exp_hi), b
    assert torch.equal(pack_q(Wq), Wp)
    assert np.array_equal(Wq.numpy(), orc.unpack_w(Wp.numpy()))


# [2] full-domain round trip in both nibble positions, boundaries
def test_value_roundtrip_all_positions():
    v = torch.arange(-8, 8, dtype=torch.int32)
    even = torch.zeros(32, dtype=torch.int32)
    even[0::2] = v
    odd = torch.zeros(32, dtype=torch.int32)
    odd[1::2] = v
    assert torch.equal(unpack_w(pack_q(even.view(1, -1)))[0, 0::2], v)
    assert torch.equal(unpack_w(pack_q(odd.view(1, -1)))[0, 1::2], v)
    b = torch.tensor([-7, 0, 7], dtype=torch.int32)
    e = torch.zeros(6, dtype=torch.int32)
    e[0::2] = b
    o = torch.zeros(6, dtype=torch.int32)
    o[1::2] = b
    assert torch.equal(unpack_w(pack_q(e.view(1, -1)))[0, 0::2], b)
    assert torch.equal(unpack_w(pack_q(o.view(1, -1)))[0, 1::2], b)


# [3] quantizer contract
def test_quantizer_contract():
    torch.manual_seed(0)
    N, G, K = 4, 3, 384
    W = (torch.randn(N, K) * 0.5).to(torch.float16)
    W.view(N, G, GROUP_SIZE)[:, 1, :].fill_(0)
    Wp, s16 = quantize_w(W)
    assert tuple(Wp.shape) == (N, K // 2) and Wp.dtype == torch.uint8
    assert tuple(s16.shape) == (N, G) and s16.dtype == torch.float16
    Wq = unpack_w(Wp)
    assert int(Wq.abs().max()) <= INT4_MAX
    assert torch.equal(s16[2, 1:2], torch.zeros(1, dtype=torch.float16))
    assert bool((Wq[2, 128:256] == 0).all())
    Wg = W.float().view(N, G, GROUP_SIZE)
    amax = Wg.abs().amax(dim=2)
    assert torch.equal(s16, (amax / 7).to(torch.float16))
    s32 = amax / 7
    q_ref = torch.round(Wg / s32.unsqueeze(2)).clamp_(-7, 7)
    q_ref = torch.where(s32.unsqueeze(2) == 0, torch.zeros_like(q_ref), q_ref)
    assert torch.equal(Wq.view(N, G, GROUP_SIZE), q_ref.to(torch.int32))
    s32c = torch.where(s32 == 0, torch.ones_like(s32), s32)
    err = (Wg - q_ref * s32c.unsqueeze(2)).abs()
    assert bool((err <= 0.5 * s32c.unsqueeze(2) + 1e-6).all())
    Wz = torch.zeros(2, K, dtype=torch.float16)
    Wpz, sz = quantize_w(Wz)
    assert bool((sz == 0).all()) and bool((Wpz == 0).all())
    assert bool(torch.isfinite(sz).all())


def test_quantizer_matches_oracle_bit_for_bit():
    rng = np.random.default_rng(31)
    for scale in (0.02, 1.0, 1e-4, 10.0):
        W = (rng.standard_normal((9, 640)) * scale).astype(np.float16)
        W[3, 128:256] = 0
        Wp, s = quantize_w(torch.from_numpy(W))
        wp_n, s_n = orc.quantize_w4(W)
        wp_c, s_c = orc.quantize_w4_c(W)
        assert np.array_equal(Wp.numpy(), wp_n) and np.array_equal(Wp.numpy(), wp_c)
        assert np.array_equal(s.numpy().view(np.uint16), s_n.view(np.uint16))
        assert np.array_equal(s.numpy().view(np.uint16), s_c.view(np.uint16))
    # exact ties round half to even
    W = np.zeros((1, 128), np.float16)
    W[0, :8] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]
    Wp, _ = quantize_w(torch.from_numpy(W))
    assert unpack_w(Wp)[0, :8].tolist() == [7, 0, 2, 2, 0, -2, -2, 4]


# [4] rejection paths raise ValueError
@pytest.mark.parametrize("make", [
    lambda: quantize_w(torch.randn(2, 256, dtype=torch.float16).view(-1)),
    lambda: quantize_w(torch.randn(2, 256, dtype=torch.float16).view(2, 2, 128)),
    lambda: quantize_w(torch.randn(2, 256)),
    lambda: quantize_w(torch.randn(256, 2, dtype=torch.float16).t()),
    lambda: quantize_w(torch.randn(2, 200, dtype=torch.float16)),
    lambda: pack_q(torch.zeros(1, 3, dtype=torch.int32)),
    lambda: pack_q(torch.tensor([[8, 0]], dtype=torch.int32)),
    lambda: pack_q(torch.tensor([[-9, 0]], dtype=torch.int32)),
    lambda: unpack_w(torch.zeros(4, dtype=torch.uint8)),
    lambda: unpack_w(torch.zeros(2, 4, dtype=torch.int8)),
])
def test_rejections(make):
    with pytest.raises(ValueError):
        make()


@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_rejects_nonfinite(bad):
    W = torch.randn(2, 256, dtype=torch.float16)
    W[1, 5] = bad
    with pytest.raises(ValueError):
        quantize_w(W)


# [5] fidelity sanity
def test_fidelity_small():
    torch.manual_seed(1)
    N, K = 4, 256
    W = torch.randn(N, K, dtype=torch.float16)
    x = torch.randn(K, dtype=torch.float16)
    Wp, s16 = quantize_w(W)
    fid = fidelity_metrics(W, x, Wp, s16)
    assert all(math.isfinite(fid[k]) for k in
               ("max_abs", "rmse", "max_dequant_abs_err", "max_dequant_step_err"))
    assert fid["cosine"] is not None and 0.9 < fid["cosine"] <= 1.0 + 1e-9
    assert fid["max_dequant_step_err"] < 0.52
    assert fidelity_metrics(W, torch.zeros(K, dtype=torch.float16), Wp, s16)["cosine"] is None
    Wz = torch.zeros(N, K, dtype=torch.float16)
    Wpz, sz = quantize_w(Wz)
    fz = fidelity_metrics(Wz, x, Wpz, sz)
    assert fz["cosine"] is None and fz["max_abs"] == 0.0


# [6] dequantize reads the stored fp16 scale
def test_dequantize_uses_stored_fp16_scale():
    N, G, K = 2, 2, 256
    Wq = torch.randint(-7, 8, (N, K), dtype=torch.int32)
    Wp = pack_q(Wq)
    s16 = (torch.rand(N, G) * 0.1 + 0.01).to(torch.float16)
    Wd = dequantize_w(Wp, s16)
    assert torch.equal(Wd, Wq.float() * s16.float().repeat_interleave(GROUP_SIZE, dim=1))
    assert np.array_equal(Wd.numpy(), orc.dequantize_w4(Wp.numpy(), s16.numpy()))
    with pytest.raises(ValueError):
        dequantize_w(Wp, s16[:, :1])
