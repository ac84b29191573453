"""GPU parity tests of the FP16/FP32 GEMV (through the C ABI), checked
against the CPU oracle: the fixed accumulation bound (TOL_K = 2,
2K roundings) for every variant, dtype, shape and input mode; bit-exact
properties at full size; the reference's negative suite for every
variant; bit-identity of the scalar fallback."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
DTYPES = (torch.float16, torch.float32)
EDGE = [(1, 1), (1, 4096), (4096, 1), (16, 13), (8, 7)]
BENCH = [(1024, 4096), (4096, 1024), (4096, 4096), (11008, 4096),
         (4096, 11008)]
# (3, 16376): the largest fp16 K whose x fits the 64 KiB LDS stage is 32760;
# (5, 16380) fp32 uses exactly 64 KiB; (2, 32768) fp16 is past the limit and
# takes the K-tiled kernel; (4099, 4096) has a partial last workgroup.
# (4099, 4096), (4097, 1024), (4097, 11008): partial last workgroups of the
# 512-thread plans, with register batches of 8, 2 and 8 (three batches) chunks
EXTRA = [(3, 16376), (5, 16380), (2, 32768), (4099, 4096), (33, 1000),
         (17, 24), (4097, 1024), (4097, 11008)]
VARIANTS = ("gemv_baseline", "gemv_cdna4", "gemv_lds_tiled", "gemv_splitk4")


@pytest.fixture(scope="module")
def extg(cuda):
    from cudalab_amd.build import build
    return build("gemv")


def _inputs(N, K, dtype, mode, seed=0):
    from cudalab_amd.operators.gemv import make_w, make_x
    return (make_w(N, K, dtype, seed=seed, mode=mode, large=10.0),
            make_x(K, dtype, seed=seed + 1, mode=mode, large=10.0))


def _np(t):
    return t.detach().cpu().numpy()


def test_registry(extg):
    assert extg.variants() == ["gemv_baseline", "gemv_cdna4", "gemv_lds_tiled"]
    assert extg.quarantined_variants() == ["gemv_splitk4"]
    assert extg.aliases() == {"gemv_vec4_row": "gemv_cdna4",
                              "gemv_warp_vec4": "gemv_cdna4"}


@pytest.mark.parametrize("dtype", DTYPES, ids=["f16", "f32"])
@pytest.mark.parametrize("N,K", EDGE + BENCH + EXTRA)
def test_bound_all_variants_all_modes(extg, N, K, dtype):
    from cudalab_amd.gemv_correctness import arith_ratio
    dn = str(dtype).split(".")[-1]
    for mode in MODES:
        W, x = _inputs(N, K, dtype, mode)
        ex, S = orc.exact_gemv(_np(W), _np(x))
        if np.abs(ex).max() >= float(torch.finfo(dtype).max):
            continue        # the exact result itself overflows the dtype
        for v in VARIANTS:
            announce(f"gemv bound {v} {dn} N={N} K={K} mode={mode}")
            y = extg.forward(v, W, x)
            torch.cuda.synchronize()
            yn = _np(y)
            assert y.dtype == dtype
            assert np.all(np.isfinite(yn)), (v, mode)
            r = orc.arith_ratio_gemv(yn, ex, S, K, yn.dtype)
            assert r.max() <= 1.0, (v, dn, N, K, mode, float(r.max()))
            r_suite, _, _ = arith_ratio(y, W, x, dn)
            assert r_suite <= 1.0, (v, mode, r_suite)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f16", "f32"])
@pytest.mark.parametrize("N,K", [(4096, 4096), (11008, 4096), (4096, 11008)])
def test_full_size_bit_exact_properties(extg, N, K, dtype):
    """Determinism, y(-x) = -y(x), y(2x) = 2y(x) and row-permutation
    equivariance, bit-exact."""
    W, x = _inputs(N, K, dtype, "normal", seed=5)
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(1)).cuda()
    for v in ("gemv_cdna4", "gemv_baseline"):
        announce(f"gemv properties {v} {dtype} N={N} K={K}")
        y = extg.forward(v, W, x)
        assert torch.equal(y, extg.forward(v, W, x)), v
        assert torch.equal(extg.forward(v, W, -x), -y), v
        assert torch.equal(extg.forward(v, W, x * 2), y * 2), v
        assert torch.equal(extg.forward(v, W[perm].contiguous(), x), y[perm]), v


@pytest.mark.parametrize("dtype", DTYPES, ids=["f16", "f32"])
@pytest.mark.parametrize("N,K", [(4096, 4096), (33, 1024)])
def test_misaligned_fallback_bit_identical(extg, N, K, dtype):
    """W one element past a 16-byte boundary, x one element past one, and
    both together: every variant takes the scalar kernel, bit-identical to
    gemv_baseline, and within the bound."""
    W, x = _inputs(N, K, dtype, "normal", seed=9)
    bw = torch.zeros(W.numel() + 64, dtype=dtype, device="cuda")
    bx = torch.zeros(K + 32, dtype=dtype, device="cuda")
    W2 = bw[1:1 + W.numel()].view(N, K)
    W2.copy_(W)
    x2 = bx[1:1 + K]
    x2.copy_(x)
    assert not extg.contract_ok(W2, x) and not extg.contract_ok(W, x2)
    ex, S = orc.exact_gemv(_np(W), _np(x))
    for (Wa, xa) in ((W2, x2), (W2, x), (W, x2)):
        base = extg.forward("gemv_baseline", Wa, xa)
        for v in VARIANTS:
            announce(f"gemv fallback {v} {dtype} N={N} K={K}")
            assert torch.equal(extg.forward(v, Wa, xa), base), v
        assert orc.arith_ratio_gemv(_np(base), ex, S, K, _np(base).dtype).max() <= 1.0


@pytest.mark.parametrize("variant", VARIANTS)
def test_negative_suite(extg, variant, tmp_path):
    from cudalab_amd.gemv_negative import run_negative_suite
    announce(f"gemv negative {variant}")
    doc = run_negative_suite(extg, out_path=tmp_path / "neg.json", variant=variant)
    bad = [c for c in doc["cases"] if not c.get("pass")]
    assert not bad, bad
    assert doc["summary"]["n_total"] == 24 and doc["summary"]["all_pass"]


def test_product_suite_incumbent(extg, tmp_path):
    from cudalab_amd.operators import get
    announce("gemv product suite gemv_cdna4")
    res = get("gemv").run_correctness(extg, "gemv_cdna4", out_dir=tmp_path)
    assert res["all_pass"], res["summary"]
    assert res["summary"]["n_total"] == 100


def test_native_and_pool_timing(extg):
    from cudalab_amd.ext import pool_timing
    for dtype in DTYPES:
        W, x = _inputs(512, 4096, dtype, "normal")
        out = torch.empty(512, dtype=dtype, device="cuda")
        t = extg.native_timing("gemv_cdna4", W, x, out, warmup=5, n_windows=3,
                               launches_per_window=4)
        assert t["median_us"] > 0 and len(t["window_median_us"]) == 3
        r = pool_timing("gemv", "gemv_cdna4", [(W, x, out)], warmup=2,
                        n_launches=8, per_kernel=False)
        assert r["total_us"] > 0
        ex, S = orc.exact_gemv(_np(W), _np(x))
        assert orc.arith_ratio_gemv(_np(out), ex, S, 4096, _np(out).dtype).max() <= 1.0
