"""GPU tests of the K-tiled LDS kernels (int4gemv / qgemv): rows longer than
16384 elements, which the CDNA4 incumbents now run vectorized instead of
on the scalar kernel.

* the fixed accumulation bound (TOL_K = 2) against the oracle's exact
  values, at k from 16400 to 131072, in every input mode, for the
  incumbent (which plans the tiled kernel there) and the scalar baseline;
* bit-identity with the untiled LDS kernel of the same lane order
  (*_lds_r1 with 64 lanes per row) at k <= 16384, where the *_lds_tiled
  variants force the tiled kernel: each lane takes the same chunks in the
  same order, so the sums are the same bit for bit;
* grouped calls at large k (one launch per problem) match single calls.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
INT4_LARGE_K = [(64, 16512), (300, 20480), (4097, 28672), (33, 65536), (2, 131072)]
Q8_LARGE_K = [(7, 16400), (64, 20480), (300, 28672), (4097, 28672), (33, 65536)]
# shapes at which *_lds_r1 runs 64 lanes per row (k/32 > 32 for INT4, k/16 >
# 32 for INT8): the untiled kernel with the tiled kernel's lane order
INT4_SAME_ORDER = [(4096, 4096), (300, 16384), (77, 2048), (4097, 11008), (1, 1152)]
Q8_SAME_ORDER = [(4096, 4096), (300, 16384), (33, 11008), (4099, 1024), (2, 528)]


def _np(t):
    return t.detach().cpu().numpy()


def _check_bound(y, ex, S, K, what, ratio=None):
    """Rows whose exact value fits fp16 pass the bound (`ratio`, default the
    INT4/INT8 one); rows clearly past the fp16 range (|exact| >= 65520,
    where round-to-nearest gives inf, with a margin for the accumulation
    error) are inf of the right sign."""
    ratio = ratio or orc.arith_ratio
    yn = _np(y).astype(np.float64)
    fits = np.abs(ex) <= 65504.0
    over = np.abs(ex) >= 65520.0 * (1 + 1e-3)
    r = ratio(_np(y)[fits], ex[fits], S[fits], K)
    assert np.all(np.isfinite(yn[fits])) and (r.size == 0 or r.max() <= 1.0), \
        (what, float(r.max()) if r.size else None)
    assert np.all(np.isinf(yn[over]) & (np.sign(yn[over]) == np.sign(ex[over]))), what


def _int4(N, K, mode, seed):
    from cudalab_amd.operators.int4gemv import make_w4, make_x4
    wp, s, _ = make_w4(N, K, seed=seed, mode=mode)
    return wp, s, make_x4(K, seed=seed + 1, mode=mode)


def _q8(N, K, mode, seed):
    from cudalab_amd.operators.qgemv import make_w_q, make_x_q
    wq, s, _ = make_w_q(N, K, seed=seed, mode=mode)
    return wq, s, make_x_q(K, seed=seed + 1, mode=mode)


@pytest.mark.parametrize("N,K", INT4_LARGE_K)
def test_int4_large_k_bound(ext4, N, K):
    d = ext4.describe("int4gemv_cdna4", *_int4(1, K, "normal", 0)[::2])
    assert d["kernel"] == "tiled"
    for mode in MODES:
        wp, s, x = _int4(N, K, mode, seed=3)
        ex, S = orc.exact_w4(_np(wp), _np(s), _np(x))
        for v in ("int4gemv_cdna4", "int4gemv_lds_tiled", "int4gemv_baseline"):
            announce(f"int4 tiled bound {v} N={N} K={K} mode={mode}")
            y = ext4.forward(v, wp, s, x)
            torch.cuda.synchronize()
            _check_bound(y, ex, S, K, (v, mode))
        if mode == "zeros":
            assert not ext4.forward("int4gemv_cdna4", wp, s, x).any()


@pytest.mark.parametrize("N,K", Q8_LARGE_K)
def test_q8_large_k_bound(ext8, N, K):
    for mode in MODES:
        wq, s, x = _q8(N, K, mode, seed=4)
        if mode == "normal":
            assert ext8.describe("qgemv_cdna4", wq, x)["kernel"] == "tiled"
        ex, S = orc.exact_w8(_np(wq), _np(s), _np(x))
        for v in ("qgemv_cdna4", "qgemv_lds_tiled", "qgemv_baseline"):
            announce(f"q8 tiled bound {v} N={N} K={K} mode={mode}")
            y = ext8.forward(v, wq, s, x)
            torch.cuda.synchronize()
            _check_bound(y, ex, S, K, (v, mode))


@pytest.mark.parametrize("N,K", INT4_SAME_ORDER)
def test_int4_tiled_matches_untiled_lane_order(ext4, N, K):
    for mode in ("normal", "large", "mixed_sign"):
        wp, s, x = _int4(N, K, mode, seed=7)
        d = ext4.describe("int4gemv_lds_r1", wp, x)
        assert (d["kernel"], d["cw"], d["r"]) == ("lds", "64", "1")
        assert ext4.describe("int4gemv_lds_tiled", wp, x)["kernel"] == "tiled"
        announce(f"int4 tiled == lds_r1 N={N} K={K} mode={mode}")
        a = ext4.forward("int4gemv_lds_tiled", wp, s, x)
        b = ext4.forward("int4gemv_lds_r1", wp, s, x)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (N, K, mode)


@pytest.mark.parametrize("N,K", Q8_SAME_ORDER)
def test_q8_tiled_matches_untiled_lane_order(ext8, N, K):
    for mode in ("normal", "large", "mixed_sign"):
        wq, s, x = _q8(N, K, mode, seed=8)
        d = ext8.describe("qgemv_lds_r1", wq, x)
        assert (d["kernel"], d["cw"], d["r"]) == ("lds", "64", "1")
        announce(f"q8 tiled == lds_r1 N={N} K={K} mode={mode}")
        a = ext8.forward("qgemv_lds_tiled", wq, s, x)
        b = ext8.forward("qgemv_lds_r1", wq, s, x)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (N, K, mode)


def test_large_k_grouped_and_side_stream(ext4, ext8):
    """Grouped calls at k > 16384 run problem by problem on the tiled kernel
    and match single calls; a call on a side stream matches one on the
    default stream."""
    announce("tiled grouped + side stream")
    probs = [_int4(N, 20480, "normal", seed=20 + i) for i, N in enumerate((64, 300, 1))]
    outs = [torch.full((p[0].size(0),), float("nan"), dtype=torch.float16, device="cuda")
            for p in probs]
    ext4.forward_grouped("int4gemv_cdna4", [(w, s, x, o) for (w, s, x), o in zip(probs, outs)])
    for (w, s, x), o in zip(probs, outs):
        assert torch.equal(o, ext4.forward("int4gemv_cdna4", w, s, x))
    qprobs = [_q8(N, 28672, "normal", seed=30 + i) for i, N in enumerate((17, 200))]
    qouts = [torch.empty(p[0].size(0), dtype=torch.float16, device="cuda") for p in qprobs]
    ext8.forward_grouped("qgemv_cdna4", [(w, s, x, o) for (w, s, x), o in zip(qprobs, qouts)])
    for (w, s, x), o in zip(qprobs, qouts):
        assert torch.equal(o, ext8.forward("qgemv_cdna4", w, s, x))
    w, s, x = probs[1]
    ref = ext4.forward("int4gemv_cdna4", w, s, x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y = ext4.forward("int4gemv_cdna4", w, s, x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


# FP16/FP32 GEMV: x above the 64 KiB LDS stage (k > 32760 fp16, > 16380
# fp32) runs the K-tiled kernel; gemv_lds_tiled forces it at any k.
GEMV_LARGE_K = [(torch.float16, 2, 32768), (torch.float16, 300, 40000),
                (torch.float16, 33, 65536), (torch.float32, 64, 20000),
                (torch.float32, 5, 16388)]
# shapes at which gemv_cdna4 runs 64 lanes per row (more than 32 chunks)
GEMV_SAME_ORDER = [(torch.float16, 4096, 4096), (torch.float16, 300, 16376),
                   (torch.float16, 33, 1000), (torch.float16, 4097, 11008),
                   (torch.float32, 4096, 4096), (torch.float32, 77, 16380)]


@pytest.fixture(scope="module")
def extg(cuda):
    from cudalab_amd.build import build
    return build("gemv")


def _gemv(N, K, dtype, mode, seed):
    from cudalab_amd.operators.gemv import make_w, make_x
    return (make_w(N, K, dtype, seed=seed, mode=mode, large=10.0),
            make_x(K, dtype, seed=seed + 1, mode=mode, large=10.0))


@pytest.mark.parametrize("dtype,N,K", GEMV_LARGE_K,
                         ids=[f"{str(d)[-7:]}-{n}x{k}" for d, n, k in GEMV_LARGE_K])
def test_gemv_large_k_bound(extg, dtype, N, K):
    for mode in MODES:
        W, x = _gemv(N, K, dtype, mode, seed=5)
        if mode == "normal":
            assert extg.describe("gemv_cdna4", W, x)["kernel"] == "tiled"
        ex, S = orc.exact_gemv(_np(W), _np(x))
        for v in ("gemv_cdna4", "gemv_lds_tiled", "gemv_baseline"):
            announce(f"gemv tiled bound {v} {dtype} N={N} K={K} mode={mode}")
            y = extg.forward(v, W, x)
            torch.cuda.synchronize()
            yn = _np(y)
            if dtype == torch.float16:
                _check_bound(y, ex, S, K, (v, mode),
                             ratio=lambda a, e, s_, k: orc.arith_ratio_gemv(a, e, s_, k, np.float16))
            else:
                r = orc.arith_ratio_gemv(yn, ex, S, K, yn.dtype)
                assert np.all(np.isfinite(yn)) and r.max() <= 1.0, (v, mode, float(r.max()))


@pytest.mark.parametrize("dtype,N,K", GEMV_SAME_ORDER,
                         ids=[f"{str(d)[-7:]}-{n}x{k}" for d, n, k in GEMV_SAME_ORDER])
def test_gemv_tiled_matches_untiled_lane_order(extg, dtype, N, K):
    for mode in ("normal", "large", "mixed_sign"):
        W, x = _gemv(N, K, dtype, mode, seed=6)
        d = extg.describe("gemv_cdna4", W, x)
        assert (d["kernel"], d["cw"]) == ("lds", "64")
        announce(f"gemv tiled == cdna4 {dtype} N={N} K={K} mode={mode}")
        a = extg.forward("gemv_lds_tiled", W, x)
        b = extg.forward("gemv_cdna4", W, x)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), (dtype, N, K, mode)


@pytest.mark.parametrize("op", ["int4gemv", "qgemv", "gemv"])
def test_weights_of_4gib_or_more(op, ext4, ext8, extg):
    """W of just over 4 GiB with short rows (k = 8192): the untiled kernels'
    32-bit offsets cannot reach it, so the incumbents plan the tiled kernel
    (64-bit row bases).  Rows on both sides of the 4 GiB byte mark, and the
    first and last rows, are checked against the oracle (sampled rows only:
    the whole matrix is not copied to the host)."""
    K = 8192
    row_bytes = {"int4gemv": K // 2, "qgemv": K, "gemv": 2 * K}[op]
    first_past = (1 << 32) // row_bytes          # first row starting at or past 4 GiB
    N = first_past + 3
    g = torch.Generator(device="cuda").manual_seed(11)
    announce(f"{op} weights of 4 GiB or more: N={N} K={K}")
    x = torch.randn(K, device="cuda", generator=g).half()
    rows = torch.tensor([0, 1, N // 2, first_past - 2, first_past - 1, first_past,
                         first_past + 1, N - 1], device="cuda")
    if op == "int4gemv":
        W = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device="cuda", generator=g)
        s = (torch.rand(N, K // 128, device="cuda", generator=g) * 1e-2 + 1e-3).half()
        ext, args = ext4, (W, s, x)
        assert ext.describe("int4gemv_cdna4", W, x)["kernel"] == "tiled"
        ex, S = orc.exact_w4(_np(W[rows]), _np(s[rows]), _np(x))
        ratio = orc.arith_ratio
        variants = ("int4gemv_cdna4", "int4gemv_baseline")
    elif op == "qgemv":
        W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
        s = torch.rand(N, device="cuda", generator=g) * 1e-2 + 1e-3
        ext, args = ext8, (W, s, x)
        assert ext.describe("qgemv_cdna4", W, x)["kernel"] == "tiled"
        ex, S = orc.exact_w8(_np(W[rows]), _np(s[rows]), _np(x))
        ratio = orc.arith_ratio
        variants = ("qgemv_cdna4", "qgemv_baseline")
    else:
        W = (torch.randn(N, K, device="cuda", generator=g, dtype=torch.float16) * 0.02)
        ext, args = extg, (W, x)
        assert ext.describe("gemv_cdna4", W, x)["kernel"] == "tiled"
        ex, S = orc.exact_gemv(_np(W[rows]), _np(x))
        ratio = lambda a, e, s_, k: orc.arith_ratio_gemv(a, e, s_, k, np.float16)  # noqa: E731
        variants = ("gemv_cdna4", "gemv_baseline")
    assert W.numel() * W.element_size() > (1 << 32)
    for v in variants:
        announce(f"{op} 4 GiB weights {v}")
        y = ext.forward(v, *args)
        torch.cuda.synchronize()
        yr = _np(y[rows])
        assert np.all(np.isfinite(yr)), v
        r = ratio(yr, ex, S, K)
        assert r.max() <= 1.0, (v, float(r.max()))
    del W, args
    torch.cuda.empty_cache()
