"""GPU parity tests of the INT8 W8A16 GEMV (through the C ABI), checked
against the CPU oracle, as for INT4."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
EDGE = [(1, 1), (1, 4096), (4096, 1), (16, 13), (8, 7)]
BENCH = [(1024, 4096), (4096, 1024), (4096, 4096), (11008, 4096),
         (4096, 11008)]
# (1001, 4096): a grid (251 workgroups) that is not a multiple of the 8 XCDs
# (4097, 11008): partial last workgroup of a 512-thread plan (8+ chunks per lane)
EXTRA = [(5, 16384), (3, 16400), (17, 16), (9, 48), (300, 1040), (2, 8192),
         (1001, 4096), (4097, 11008)]


def _np(t):
    return t.detach().cpu().numpy()


def _inputs(N, K, mode, seed=0):
    from cudalab_amd.operators.qgemv import make_w_q, make_x_q
    wq, s, _ = make_w_q(N, K, seed=seed, mode=mode)
    x = make_x_q(K, seed=seed + 1, mode=mode)
    return wq, s, x


def test_registry(ext8):
    v = ext8.variants()
    assert "qgemv_baseline" in v and "qgemv_cdna4" in v
    assert ext8.aliases()["qgemv_vec16_row"] == "qgemv_cdna4"


@pytest.mark.parametrize("N,K", EDGE + BENCH + EXTRA)
def test_bound_all_variants_all_modes(ext8, N, K):
    from cudalab_amd.qgemv_correctness import arith_ratio
    for mode in MODES:
        wq, s, x = _inputs(N, K, mode)
        ex, S = orc.exact_w8(_np(wq), _np(s), _np(x))
        for v in ext8.variants():
            announce(f"int8 bound {v} N={N} K={K} mode={mode}")
            y = ext8.forward(v, wq, s, x)
            torch.cuda.synchronize()
            yn = _np(y)
            assert np.all(np.isfinite(yn)), (v, mode)
            r = orc.arith_ratio(yn, ex, S, K)
            assert r.max() <= 1.0, (v, N, K, mode, float(r.max()))
            r_suite, _, _ = arith_ratio(y, wq, s, x, "float16")
            assert r_suite <= 1.0, (v, mode, r_suite)


@pytest.mark.parametrize("N,K", BENCH)
def test_full_size_bit_exact_properties(ext8, N, K):
    wq, s, x = _inputs(N, K, "normal", seed=5)
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(1)).cuda()
    for v in ("qgemv_cdna4", "qgemv_wave_r1", "qgemv_baseline"):
        announce(f"int8 properties {v} N={N} K={K}")
        y = ext8.forward(v, wq, s, x)
        assert torch.equal(y, ext8.forward(v, wq, s, x)), v
        assert torch.equal(ext8.forward(v, wq, s, -x), -y), v
        assert torch.equal(ext8.forward(v, wq, s, x * 2), y * 2), v
        yp = ext8.forward(v, wq[perm].contiguous(), s[perm].contiguous(), x)
        assert torch.equal(yp, y[perm]), v


LDS_VARIANTS = ("qgemv_cdna4", "qgemv_lds_r1", "qgemv_lds_r2", "qgemv_lds_r4")


@pytest.mark.parametrize("N,K", EDGE + BENCH + EXTRA)
def test_lds_variants_bit_identical(ext8, N, K):
    """The LDS kernels sum each row in one lane segment, chunk by chunk in the
    same order, whatever the rows per lane and workgroup size (and past
    k = 16384 the K-tiled kernel keeps that order): every LDS variant gives
    the same bits, including lanes past the row end (clamped last chunk
    against the zero column of x) and partial last workgroups."""
    for mode in ("normal", "mixed_sign", "large"):
        w, s, x = _inputs(N, K, mode, seed=3)
        ref = ext8.forward("qgemv_lds_r1", w, s, x)
        for v in LDS_VARIANTS:
            announce(f"int8 lds identity {v} N={N} K={K} mode={mode}")
            y = ext8.forward(v, w, s, x)
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), (v, N, K, mode)


@pytest.mark.parametrize("N,K", [(4096, 4096), (64, 13), (11008, 4096)])
def test_misaligned_fallback_bit_identical(ext8, N, K):
    wq, s, x = _inputs(N, K, "normal", seed=9)
    bw = torch.zeros(wq.numel() + 64, dtype=torch.int8, device="cuda")
    bx = torch.zeros(K + 32, dtype=torch.float16, device="cuda")
    wq2 = bw[2:2 + wq.numel()].view(N, K)
    wq2.copy_(wq)
    x2 = bx[1:1 + K]
    x2.copy_(x)
    for (Wa, xa) in ((wq2, x2), (wq2, x), (wq, x2)):
        base = ext8.forward("qgemv_baseline", Wa, s, xa)
        for v in ext8.variants():
            announce(f"int8 fallback {v} N={N} K={K}")
            assert torch.equal(ext8.forward(v, Wa, s, xa), base), v
        ex, S = orc.exact_w8(_np(wq), _np(s), _np(x))
        assert orc.arith_ratio(_np(base), ex, S, K).max() <= 1.0


def test_golden_fixtures(ext8):
    from pathlib import Path
    d = np.load(Path(__file__).parent / "golden" / "qgemv_golden.npz")
    for i in range(int(d["n_cases"])):
        wq = torch.from_numpy(d[f"wq_{i}"]).cuda()
        s = torch.from_numpy(d[f"scale_{i}"]).cuda()
        x = torch.from_numpy(d[f"x_{i}"].view(np.float16)).cuda()
        for v in ext8.variants():
            y = _np(ext8.forward(v, wq, s, x))
            r = orc.arith_ratio(y, d[f"exact_{i}"], d[f"S_{i}"], x.numel())
            assert r.max() <= 1.0, (i, v)


@pytest.mark.parametrize("variant", ["qgemv_baseline", "qgemv_cdna4",
                                     "qgemv_wave_r1", "qgemv_wave_r2",
                                     "qgemv_wave_r4"])
def test_negative_suite(ext8, variant, tmp_path):
    from cudalab_amd.qgemv_negative import run_negative_suite
    announce(f"int8 negative suite {variant}")
    doc = run_negative_suite(ext8, out_path=tmp_path / "neg.json",
                             variant=variant)
    bad = [c for c in doc["cases"] if not c.get("pass")]
    assert doc["summary"]["all_pass"], bad
    assert doc["summary"]["n_total"] == 29


def test_product_suite_incumbent(ext8, tmp_path):
    from cudalab_amd.operators import get
    announce("int8 product correctness suite")
    r = get("qgemv").run_correctness(ext8, "qgemv_cdna4", out_dir=tmp_path)
    assert r["all_pass"], r["summary"]["failed"]
    assert r["summary"]["n_total"] == 50
    _check_fidelity(tmp_path / "quantization_fidelity.json")


# The reference's archived layer-(c) record
# (experiments/qgemv/correctness/v0.6/quantization_fidelity.json): min cosine
# 0.9998970268657201, max step error 0.5000019073486328, max |q| 127.
REF_MIN_COSINE = 0.9998970268657201


def _check_fidelity(path):
    """Layer (c) asserted: max |q| is 127; the step error |W - q*s| / s of
    the fp32 per-row scale is 1/2 plus FP32 rounding of W/s and q*s (at most
    128 * 2^-24 each way); the cosine is no worse than the reference's
    archived minimum."""
    import json
    d = json.loads(path.read_text())
    summ, cases = d["summary"], d["cases"]
    assert summ["n_cases"] == 25 and summ["max_abs_q"] == 127
    for c in cases:
        if c["mode"] == "zeros":
            assert c["max_abs_q"] == 0 and c["cosine"] is None
            continue
        assert c["max_abs_q"] == 127, c
        assert c["max_dequant_step_err"] <= 0.5 + 2 * 128 * 2.0 ** -24, c
    assert summ["min_cosine"] >= REF_MIN_COSINE, summ
