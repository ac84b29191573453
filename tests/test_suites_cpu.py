"""Consistency of the product's torch-based suite arithmetic with the CPU
oracle, generator determinism, bench helpers -- all on CPU."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import torch

from cudalab_amd import int4gemv_correctness as c4
from cudalab_amd import qgemv_correctness as c8
from cudalab_amd.evaluator.bench import BenchPool, cold_pool_sets
from cudalab_amd.operators.gemv import make_w, make_x
from cudalab_amd.operators.int4gemv import int4_bytes, make_w4, make_x4
from cudalab_amd.operators.qgemv import make_w_q, make_x_q, q8_bytes
from oracle import oracle as orc

ROOT = Path(__file__).resolve().parents[1]


def test_ulp_matches_oracle():
    v = torch.tensor([0.0, 1e-8, 6.1e-5, 1.0, -3.5, 1000.0, 65504.0])
    assert np.array_equal(c4._ulp(v, "float16").numpy().astype(np.float64),
                          orc.ulp16(v.numpy()))


def test_suite_bound_matches_oracle_bound():
    """The suite's fp64 torch bound and the oracle's exact-integer bound
    give the same ratio on the same output (up to fp64 rounding of the
    exact value)."""
    for mode in ("normal", "mixed_sign", "tiny", "large"):
        wp, s, _ = make_w4(16, 512, seed=3, mode=mode, device="cpu")
        x = make_x4(512, seed=4, mode=mode, device="cpu")
        _, y16 = orc.ref_f32_w4(wp.numpy(), s.numpy(), x.numpy())
        y = torch.from_numpy(y16.copy())
        r_suite, _, _ = c4.arith_ratio(y, wp, s, x, "float16")
        ex, S = orc.exact_w4(wp.numpy(), s.numpy(), x.numpy())
        r_orc = float(orc.arith_ratio(y16, ex, S, 512).max())
        assert abs(r_suite - r_orc) <= 1e-9 + 1e-6 * r_orc, mode
        wq, sq, _ = make_w_q(16, 77, seed=3, mode=mode, device="cpu")
        xq = make_x_q(77, seed=4, mode=mode, device="cpu")
        _, y8 = orc.ref_f32_w8(wq.numpy(), sq.numpy(), xq.numpy())
        r_suite, _, _ = c8.arith_ratio(torch.from_numpy(y8.copy()), wq, sq, xq, "float16")
        ex, S = orc.exact_w8(wq.numpy(), sq.numpy(), xq.numpy())
        r_orc = float(orc.arith_ratio(y8, ex, S, 77).max())
        assert abs(r_suite - r_orc) <= 1e-9 + 1e-6 * r_orc, mode


def test_generators_deterministic_and_modes():
    a = make_w(8, 256, torch.float16, device="cpu", seed=5, mode="mixed_sign")
    b = make_w(8, 256, torch.float16, device="cpu", seed=5, mode="mixed_sign")
    assert torch.equal(a, b)
    par = (torch.arange(8)[:, None] + torch.arange(256)[None, :]) % 2
    assert bool(((a > 0) | (a == 0))[par == 0].all())
    assert bool(((a < 0) | (a == 0))[par == 1].all())
    assert bool((make_w(4, 128, torch.float16, device="cpu", mode="zeros") == 0).all())
    t = make_x(4096, torch.float16, device="cpu", seed=1, mode="tiny")
    assert float(t.abs().max()) < 1e-3
    assert int((t.abs() < 6.1e-5).sum()) > 100          # fp16 subnormals present
    xm = make_x(4096, torch.float16, device="cpu", seed=1, mode="mixed_sign")
    assert 0.4 < float((xm < 0).float().mean()) < 0.6
    assert not torch.equal(make_x(64, torch.float16, device="cpu", seed=1),
                           make_x(64, torch.float16, device="cpu", seed=2))


def test_byte_formulas_and_pool_size():
    assert int4_bytes(4096, 4096) == 8_667_136
    assert int4_bytes(11008, 4096) == 23_279_104
    assert q8_bytes(4096, 4096) == 16_809_984
    n = cold_pool_sets(int4_bytes(4096, 4096))
    assert n * int4_bytes(4096, 4096) > 512 * 1024 * 1024
    assert cold_pool_sets(10 << 30) == 2


def test_bench_pool_validation():
    import pytest
    with pytest.raises(ValueError):
        BenchPool(xs=[1, 2], outs=[1, 2], pool_size=2, working_set_bytes=0,
                  element_size=2, mode="hot", launch=lambda *a: None)
    with pytest.raises(ValueError):
        BenchPool(xs=[1], outs=[1], pool_size=1, working_set_bytes=0,
                  element_size=2, mode="warm", launch=lambda *a: None)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "8"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_cpu_baseline_bounded_sample():
    """bench.py's CPU leg on a tiny sample: the oracle port cycles over
    distinct sets, reports medians and call counts, and its first result is
    checked against the fp64 bound before anything is timed."""
    import importlib.util
    import torch
    from cudalab_amd.int4gemv_quantize import quantize_w
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    g = torch.Generator().manual_seed(5)
    sets = []
    for _ in range(4):
        W = (torch.randn(64, 256, generator=g) * 0.02).half()
        wp, s = quantize_w(W)
        sets.append((wp, s, torch.randn(256, generator=g).half(), None))
    cpu = bench.cpu_baseline(64, 256, sets, seconds=0.05, max_sets=3)
    assert cpu["kind"] == "port" and cpu["unit"] == "GB/s" and cpu["value"] > 0
    assert cpu["cores"] >= 1 and cpu["us_per_call"] > 0
    assert "cycling over 3 distinct host-resident input sets" in cpu["sample"]
    assert cpu["c_port_1_thread_calls"] >= 5 and cpu["sample_cpu_seconds"] > 0
    t = cpu["torch_formulation_us"]
    assert min(t["calls"]) >= 3 and t["all_threads"] > 0 and t["one_thread"] > 0
