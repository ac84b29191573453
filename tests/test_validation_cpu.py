"""Host-side validation of the extension objects on CPU tensors: the
reference's check order and message substrings
(kernels/int4gemv/bindings.cpp:60-121, kernels/qgemv/bindings.cpp:65-121)
for every negative case that metadata alone decides.  CPU tensors that pass
every other check stop at the device check, so nothing is ever launched."""
from __future__ import annotations

import pytest
import torch

from cudalab_amd.build import build


@pytest.fixture(scope="module")
def e4():
    return build("int4gemv")


@pytest.fixture(scope="module")
def e8():
    return build("qgemv")


def _int4_base(N=8, K=256):
    W = torch.zeros(N, K // 2, dtype=torch.uint8)
    s = torch.zeros(N, K // 128, dtype=torch.float16)
    x = torch.zeros(K, dtype=torch.float16)
    return W, s, x


def _msg(fn):
    with pytest.raises(RuntimeError) as ei:
        fn()
    return str(ei.value)


def test_int4_cases_in_reference_order(e4):
    W, s, x = _int4_base()
    f = lambda *a: e4.forward("int4gemv_cdna4", *a)  # noqa: E731
    cases = [
        ((W.view(-1), s, x), "必须是 2 维"),
        ((W.view(2, 4, 128), s, x), "必须是 2 维"),
        ((torch.zeros(0, 128, dtype=torch.uint8), s[:0], x), "N 必须 > 0"),
        ((torch.zeros(8, 0, dtype=torch.uint8), s, x), "K/2 必须 > 0"),
        ((W.half(), s, x), "必须是 uint8"),
        ((W.to(torch.int8), s, x), "必须是 uint8"),
        ((torch.zeros(8, 32, dtype=torch.uint8), torch.zeros(8, 1, dtype=torch.float16),
          torch.zeros(64, dtype=torch.float16)), "必须可被 128 整除"),
        ((torch.zeros(32, 8, dtype=torch.uint8).t(), s, x), "必须可被 128 整除"),
        ((torch.zeros(128, 8, dtype=torch.uint8).t(), s, x), "连续内存"),
        ((W, s, x), "CUDA 张量"),
    ]
    for args, sub in cases:
        assert sub in _msg(lambda: f(*args)), sub


def test_int4_unknown_variant_first(e4):
    W, s, x = _int4_base()
    m = _msg(lambda: e4.forward("no_such_int4gemv_variant", W.view(-1), s, x))
    assert "未知 int4gemv 变体" in m and "int4gemv_cdna4" in m


def test_int4_scale_x_out_checks_follow_w(e4, monkeypatch):
    """Pretend W passes (a CPU stand-in for a GPU tensor) to reach the scale,
    x and out checks in their reference order."""
    W, s, x = _int4_base()
    monkeypatch.setattr(type(e4), "_validate_w", lambda self, Wp: None)
    f = lambda *a: e4.forward("int4gemv_cdna4", *a)  # noqa: E731
    assert "scale 组数必须等于 K/128" in _msg(lambda: f(W, s[:, :1].contiguous(), x))
    assert "scale 行数必须等于 N" in _msg(lambda: f(W, s[:7].contiguous(), x))
    assert "必须是 2 维" in _msg(lambda: f(W, s.view(-1), x))
    assert "必须是 float16" in _msg(lambda: f(W, s.float(), x))
    assert "连续内存" in _msg(lambda: f(W, torch.zeros(16, 2, dtype=torch.float16)[::2], x))
    assert "CUDA 张量" in _msg(lambda: f(W, s, x))
    monkeypatch.setattr(type(e4), "_validate_scale", lambda self, Wp, sc: None)
    assert "x 长度必须等于 K" in _msg(lambda: f(W, s, x[:128].contiguous()))
    assert "必须是 1 维" in _msg(lambda: f(W, s, x.view(1, -1)))
    assert "必须是 float16" in _msg(lambda: f(W, s, x.float()))
    assert "连续内存" in _msg(lambda: f(W, s, torch.zeros(512, dtype=torch.float16)[::2]))
    assert "CUDA 张量" in _msg(lambda: f(W, s, x))
    monkeypatch.setattr(type(e4), "_validate_x", lambda self, Wp, xx: None)
    g = lambda o: e4.forward_into("int4gemv_cdna4", W, s, x, o)  # noqa: E731
    assert "out 长度必须等于 N" in _msg(lambda: g(torch.zeros(7, dtype=torch.float16)))
    assert "必须是 1 维" in _msg(lambda: g(torch.zeros(8, 1, dtype=torch.float16)))
    assert "必须是 float16" in _msg(lambda: g(torch.zeros(8)))
    assert "连续内存" in _msg(lambda: g(torch.zeros(16, dtype=torch.float16)[::2]))
    assert "CUDA 张量" in _msg(lambda: g(torch.zeros(8, dtype=torch.float16)))


def test_int8_cases_in_reference_order(e8, monkeypatch):
    W = torch.zeros(8, 64, dtype=torch.int8)
    s = torch.zeros(8)
    x = torch.zeros(64, dtype=torch.float16)
    f = lambda *a: e8.forward("qgemv_cdna4", *a)  # noqa: E731
    assert "必须是 2 维" in _msg(lambda: f(W.view(-1), s, x))
    assert "N 必须 > 0" in _msg(lambda: f(torch.zeros(0, 64, dtype=torch.int8), s[:0], x))
    assert "K 必须 > 0" in _msg(lambda: f(torch.zeros(8, 0, dtype=torch.int8), s, x))
    assert "必须是 int8" in _msg(lambda: f(W.half(), s, x))
    assert "必须是 int8" in _msg(lambda: f(W.int(), s, x))
    assert "连续内存" in _msg(lambda: f(torch.zeros(64, 8, dtype=torch.int8).t(), s, x))
    assert "CUDA 张量" in _msg(lambda: f(W, s, x))
    assert "未知 qgemv 变体" in _msg(lambda: e8.forward("no_such_qgemv_variant", W, s, x))
    monkeypatch.setattr(type(e8), "_validate_w", lambda self, Wq: None)
    assert "scale 长度必须等于 N" in _msg(lambda: f(W, s[:7].contiguous(), x))
    assert "必须是 1 维" in _msg(lambda: f(W, s.view(8, 1), x))
    assert "必须是 float32" in _msg(lambda: f(W, s.half(), x))
    assert "连续内存" in _msg(lambda: f(W, torch.zeros(16)[::2], x))
    assert "CUDA 张量" in _msg(lambda: f(W, s, x))
    monkeypatch.setattr(type(e8), "_validate_scale", lambda self, Wq, sc: None)
    assert "x 长度必须等于 K" in _msg(lambda: f(W, s, x[:63].contiguous()))
    assert "必须是 float16" in _msg(lambda: f(W, s, x.float()))


def test_native_timing_argument_checks(e4):
    W, s, x = _int4_base()
    o = torch.zeros(8, dtype=torch.float16)
    assert "warmup 必须 >= 0" in _msg(lambda: e4.native_timing("int4gemv_cdna4", W, s, x, o, warmup=-1))
    assert "n_windows 必须 >= 1" in _msg(lambda: e4.native_timing("int4gemv_cdna4", W, s, x, o, n_windows=0))
    assert "launches_per_window 必须 >= 1" in _msg(
        lambda: e4.native_timing("int4gemv_cdna4", W, s, x, o, launches_per_window=0))
    assert "未知 int4gemv 变体" in _msg(lambda: e4.native_timing("zzz", W, s, x, o))


def test_registry_api(e4, e8):
    assert e4.variants() == sorted(e4.variants())
    assert e4.quarantined_variants() == [] and e8.quarantined_variants() == []
    assert e4.resolve("int4gemv_rowtile4_hx") == "int4gemv_cdna4"
    assert e8.resolve("qgemv_vec16_row") == "qgemv_cdna4"
    from cudalab_amd.operators import get, names
    assert names() == ["gemv", "int4gemv", "qgemv"]
    assert get("int4gemv").variants(e4) == e4.variants()
    with pytest.raises(KeyError):
        get("rmsnorm")


def test_grouped_checks(e4, monkeypatch):
    """forward_grouped checks every problem as forward_into does, and
    rejects an empty list and mixed K before anything is launched."""
    W, s, x = _int4_base()
    o = torch.zeros(8, dtype=torch.float16)
    assert "non-empty" in _msg(lambda: e4.forward_grouped("int4gemv_cdna4", []))
    assert "未知 int4gemv 变体" in _msg(lambda: e4.forward_grouped("zzz", [(W, s, x, o)]))
    assert "CUDA 张量" in _msg(lambda: e4.forward_grouped("int4gemv_cdna4", [(W, s, x, o)]))
    for name in ("_validate_w", "_validate_scale", "_validate_x", "_validate_out"):
        monkeypatch.setattr(type(e4), name, lambda self, *a: None)
    W2 = torch.zeros(8, 256, dtype=torch.uint8)
    assert "share K" in _msg(lambda: e4.forward_grouped("int4gemv_cdna4", [(W, s, x, o), (W2, s, x, o)]))


@pytest.fixture(scope="module")
def eg():
    return build("gemv")


def test_gemv_cases_in_reference_order(eg, monkeypatch):
    """kernels/gemv/bindings.cpp:87-125: W dim, N, K, dtype, contiguous,
    device; then x; then out."""
    W = torch.zeros(8, 64, dtype=torch.float16)
    x = torch.zeros(64, dtype=torch.float16)
    f = lambda *a: eg.forward("gemv_cdna4", *a)  # noqa: E731
    assert "必须是 2 维" in _msg(lambda: f(W.view(-1), x))
    assert "N 必须 > 0" in _msg(lambda: f(torch.zeros(0, 64, dtype=torch.float16), x))
    assert "K 必须 > 0" in _msg(lambda: f(torch.zeros(8, 0, dtype=torch.float16), x))
    assert "float16 / float32" in _msg(lambda: f(W.bfloat16(), x))
    assert "float16 / float32" in _msg(lambda: f(W.int(), x))
    assert "连续内存" in _msg(lambda: f(torch.zeros(64, 8, dtype=torch.float16).t(), x))
    assert "CUDA 张量" in _msg(lambda: f(W, x))
    assert "未知 gemv 变体" in _msg(lambda: eg.forward("zzz", W, x))
    m = _msg(lambda: eg.forward("zzz", W, x))
    assert "gemv_splitk4" in m and "NOT_FOR_NORMAL_DISPATCH" in m
    monkeypatch.setattr(type(eg), "_validate_w", lambda self, Wa: None)
    assert "必须是 1 维" in _msg(lambda: f(W, x.view(1, -1)))
    assert "x 长度必须等于 K" in _msg(lambda: f(W, x[:63].contiguous()))
    assert "dtype 必须与 W 一致" in _msg(lambda: f(W, x.float()))
    assert "连续内存" in _msg(lambda: f(W, torch.zeros(128, dtype=torch.float16)[::2]))
    assert "CUDA 张量" in _msg(lambda: f(W, x))
    monkeypatch.setattr(type(eg), "_validate_x", lambda self, Wa, xa: None)
    g = lambda o: eg.forward_into("gemv_cdna4", W, x, o)  # noqa: E731
    assert "out 长度必须等于 N" in _msg(lambda: g(torch.zeros(7, dtype=torch.float16)))
    assert "必须是 1 维" in _msg(lambda: g(torch.zeros(8, 1, dtype=torch.float16)))
    assert "dtype 必须与 W 一致" in _msg(lambda: g(torch.zeros(8)))
    assert "连续内存" in _msg(lambda: g(torch.zeros(16, dtype=torch.float16)[::2]))
    assert "CUDA 张量" in _msg(lambda: g(torch.zeros(8, dtype=torch.float16)))


def test_gemv_registry(eg):
    assert eg.variants() == ["gemv_baseline", "gemv_cdna4", "gemv_lds_tiled"]
    assert eg.quarantined_variants() == ["gemv_splitk4"]
    assert eg.all_variants() == ["gemv_baseline", "gemv_cdna4", "gemv_lds_tiled",
                                 "gemv_splitk4"]
    assert eg.resolve("gemv_vec4_row") == "gemv_cdna4"
    assert eg.resolve("gemv_warp_vec4") == "gemv_cdna4"
