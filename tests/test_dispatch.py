"""Dispatch tables (pure CPU).  The reference's (M, H, dtype) table keeps
its API and answers (tests/test_dispatch.py:20-115 of the reference); the
quantized-GEMV table routes every shape to the CDNA4 incumbent."""
from __future__ import annotations

import pytest
import torch

from cudalab_amd import dispatch


def test_routed_cells():
    cases = [
        (128, 4096, torch.float32, "v2_reg"),
        (128, 8192, torch.float16, "v2_reg"),
        (128, 4096, torch.float16, "v4_vec_reg"),
        (1, 1024, torch.float16, "baseline"),
        (128, 1024, torch.float16, "baseline"),
        (1, 4096, torch.float16, "baseline"),
        (16, 4096, torch.float16, "baseline"),
        (1024, 4096, torch.float16, "baseline"),
        (1, 1024, torch.float32, "baseline"),
        (128, 1024, torch.float32, "baseline"),
        (1, 4096, torch.float32, "baseline"),
        (16, 4096, torch.float32, "baseline"),
        (1024, 4096, torch.float32, "baseline"),
        (128, 8192, torch.float32, "baseline"),
        (1024, 8192, torch.float16, "baseline"),
        (16, 8192, torch.float32, "baseline"),
        (512, 2048, torch.float16, "baseline"),
    ]
    for M, H, dt, exp in cases:
        assert dispatch.select_variant(M, H, dt) == exp, (M, H, dt)


def test_table_matches_selector():
    for (M, H, dname), (v, _src, _why) in dispatch.TABLE.items():
        dt = torch.float16 if dname == "float16" else torch.float32
        assert dispatch.select_variant(M, H, dt) == v


def test_evidence_sources():
    for M, H, dt in [(128, 4096, torch.float32), (128, 8192, torch.float16)]:
        info = dispatch.dispatch_info(M, H, dt)
        assert info["evidence_source"] == "paired-evidence"
        assert info["variant"] == "v2_reg"
    info = dispatch.dispatch_info(128, 4096, torch.float16)
    assert info["evidence_source"] == "incumbent-fallback"
    assert "NO_UNIQUE_WINNER" in info["reason"]
    for M, H, dt in [(1024, 4096, torch.float16), (1, 4096, torch.float16),
                     (128, 8192, torch.float32), (128, 1024, torch.float16)]:
        assert dispatch.dispatch_info(M, H, dt)["evidence_source"] == "matrix-only"
    for M, H, dt in [(1024, 8192, torch.float16), (16, 8192, torch.float32)]:
        info = dispatch.dispatch_info(M, H, dt)
        assert info["evidence_source"] == "baseline-fallback"
        assert info["variant"] == "baseline"


def test_conflict_cell_not_claimed_stable():
    info = dispatch.dispatch_info(16, 4096, torch.float16)
    assert info["variant"] == "baseline" and "冲突" in info["reason"]


def test_unsupported_h_falls_back():
    assert dispatch.select_variant(128, 300, torch.float16) == "baseline"
    assert dispatch.select_variant(256, 512, torch.float16) == "baseline"
    assert not dispatch._supported("v4_vec_reg", 300, torch.float16)
    assert dispatch._supported("v1_vec", 8, torch.float16)


@pytest.mark.parametrize("op", ["int4gemv", "qgemv"])
def test_gemv_routing(op):
    for N, K in [(1024, 4096), (4096, 1024), (4096, 4096), (11008, 4096),
                 (4096, 11008)]:
        info = dispatch.gemv_dispatch_info(op, N, K)
        assert info["variant"] == f"{op}_cdna4"
        assert info["evidence_source"] == "incumbent"
        assert info["kernel"] == "lds" and not info["fallback"]
        assert "LDS kernel" in info["reason"]
    # past 16384 elements per row the incumbent runs the K-tiled kernel
    info = dispatch.gemv_dispatch_info(op, 8, 16512)
    assert info["evidence_source"] == "incumbent"
    assert info["kernel"] == "tiled" and "K-tiled" in info["reason"]
    assert "16512 > 16384" in info["reason"]
    with pytest.raises(KeyError):
        dispatch.select_gemv_variant("gemv", 1, 1)
    with pytest.raises(ValueError):
        dispatch.select_gemv_variant(op, 0, 128)


@pytest.mark.parametrize("op", ["int4gemv", "qgemv"])
@pytest.mark.parametrize("N,K,woff,xoff", [
    (4096, 4096, 0, 0), (11008, 4096, 0, 0), (8, 16512, 0, 0),
    (8192, 28672, 0, 0), (4096, 4096, 2, 0), (4096, 4096, 0, 2),
    (1 << 20, 8192, 0, 0),
])
def test_gemv_routing_agrees_with_the_library_plan(op, N, K, woff, xoff):
    """The routing answer is the plan the library launches for that call."""
    from cudalab_amd import _capi
    info = dispatch.gemv_dispatch_info(op, N, K, woff, xoff)
    d = _capi.describe_launch(op, f"{op}_cdna4", N, K, 4096 + woff, 8192 + xoff)
    assert info["kernel"] == d["kernel"]
    assert info["plan"] == {k: int(d[k]) for k in ("cw", "j", "r", "tile", "block", "grid")}
    assert info["fallback"] == (d["fallback"] == "1")
    assert (info["evidence_source"] == "scalar-path") == (d["kernel"] == "scalar")
    if woff or xoff:
        assert info["kernel"] == "scalar" and "alignment" in info["reason"]
        assert f"{op}_baseline" in info["reason"]
    if N == 1 << 20:    # 4 GiB of weights or more: tiled, 64-bit row bases
        big = N * (K // 2 if op == "int4gemv" else K) >= 1 << 32
        assert info["kernel"] == ("tiled" if big else "lds")
        if big:
            assert "4 GiB" in info["reason"]


def test_gemv_routing_int4_k_contract():
    with pytest.raises(ValueError):
        dispatch.select_gemv_variant("int4gemv", 8, 100)
    info = dispatch.gemv_dispatch_info("qgemv", 8, 13)
    assert info["evidence_source"] == "scalar-path" and info["kernel"] == "scalar"
    assert "k%16" in info["reason"]
