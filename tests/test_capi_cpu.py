"""The C-ABI library on CPU: it loads, exports every function that
include/*.h declares, and its host-only entry points (registry, contract
predicate, launch description, argument errors) behave -- no kernel is
launched and no GPU is needed."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from cudalab_amd import _capi

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(cq_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_header_declares_the_abi():
    names = _declared_functions()
    assert {"cq_int4gemv", "cq_qgemv", "cq_native_timing", "cq_pool_timing", "cq_read_ceiling",
            "cq_launch_floor",
            "cq_int4gemv_grouped", "cq_qgemv_grouped", "cq_gemv",
            "cq_variants", "cq_vec_contract_ok", "cq_describe_launch",
            "cq_last_error", "cq_version"} <= names


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    for name in sorted(_declared_functions()):
        assert hasattr(lib, name), name
    assert set(_capi.SIGNATURES) == _declared_functions()


def test_version_and_lists():
    assert "gfx950" in _capi.version()
    for op in ("int4gemv", "qgemv"):
        normal = _capi.variant_list(op)
        assert normal == sorted(normal)
        assert f"{op}_baseline" in normal and f"{op}_cdna4" in normal
        assert _capi.variant_list(op, _capi.CQ_LIST_ALL) == normal
        assert _capi.variant_list(op, _capi.CQ_LIST_QUARANTINED) == []
        al = _capi.aliases(op)
        assert al and all(t == f"{op}_cdna4" for t in al.values())
    assert "int4gemv_rowtile4_hx" in _capi.aliases("int4gemv")
    assert "qgemv_vec16_row" in _capi.aliases("qgemv")


def test_variants_buffer_protocol():
    lib = _capi.load()
    need = lib.cq_variants(_capi.CQ_OP_INT4GEMV, _capi.CQ_LIST_NORMAL, None, 0)
    assert need > 1
    small = ctypes.create_string_buffer(4)
    assert lib.cq_variants(_capi.CQ_OP_INT4GEMV, 0, small, 4) == need
    assert small.raw == b"\0" * 4          # nothing written when too small
    assert lib.cq_variants(7, 0, None, 0) < 0
    assert lib.cq_variants(0, 9, None, 0) < 0


def test_vector_contract_predicate():
    ok = _capi.vec_contract_ok
    assert ok("int4gemv", 0x1000, 0x2000, 4096)
    assert not ok("int4gemv", 0x1001, 0x2000, 4096)
    assert not ok("int4gemv", 0x1000, 0x2002, 4096)
    assert not ok("int4gemv", 0x1000, 0x2000, 4112)      # k % 32 != 0
    assert ok("qgemv", 0x1000, 0x2000, 16)
    assert not ok("qgemv", 0x1000, 0x2000, 13)
    assert not ok("qgemv", 0x1008, 0x2000, 64)


@pytest.mark.parametrize("n,k,kernel,cw,j,r,block", [
    (4096, 4096, "lds", 64, 2, 2, 512),
    (11008, 4096, "lds", 64, 2, 2, 512),
    (4096, 11008, "lds", 64, 6, 1, 512),      # 3+ chunks per lane: 512 threads
    (1024, 4096, "lds", 64, 2, 1, 256),
    (4096, 1024, "lds", 32, 1, 1, 256),
    (1, 128, "lds", 16, 1, 1, 256),
    (5, 16384, "lds", 64, 8, 1, 256),
    # two rows per lane but fewer than 256 workgroups at 512 threads
    (3000, 4096, "lds", 64, 2, 1, 256),
])
def test_int4_launch_plans(n, k, kernel, cw, j, r, block):
    d = _capi.describe_launch("int4gemv", "int4gemv_cdna4", n, k, 4096, 8192)
    assert (d["kernel"], int(d["cw"]), int(d["j"]), int(d["r"])) == (kernel, cw, j, r)
    assert d["fallback"] == "0" and int(d["block"]) == block
    rows_per_block = (64 // cw) * r * (block // 64)
    assert int(d["grid"]) == -(-n // rows_per_block)


def test_int4_plans_fall_back_to_scalar():
    d = _capi.describe_launch("int4gemv", "int4gemv_cdna4", 8, 4096, 4097, 8192)
    assert d["kernel"] == "scalar" and d["fallback"] == "1" and "alignment" in d["why"]
    d = _capi.describe_launch("int4gemv", "int4gemv_cdna4", 8, 16512, 4096, 8192)
    assert d["kernel"] == "scalar" and d["fallback"] == "1"
    d = _capi.describe_launch("int4gemv", "int4gemv_baseline", 8, 4096, 4096, 8192)
    assert d["kernel"] == "scalar" and d["fallback"] == "0"
    d = _capi.describe_launch("int4gemv", "int4gemv_rowtile4_hx", 8, 4096, 4096, 8192)
    assert d["variant"] == "int4gemv_cdna4" and d["kernel"] == "lds"
    # weights of 4 GiB or more would overflow the 32-bit offsets
    d = _capi.describe_launch("int4gemv", "int4gemv_cdna4", 1 << 20, 8192, 4096, 8192)
    assert d["kernel"] == "scalar" and "4 GiB" in d["why"]


def test_q8_launch_plans():
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 4096, 4096, 4096, 8192)
    assert (d["kernel"], d["cw"], d["j"], d["r"]) == ("lds", "64", "4", "1")
    assert (d["block"], d["grid"]) == ("256", "1024")
    # 8+ chunks per lane and a grid that still covers every CU: 512 threads
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 4096, 11008, 4096, 8192)
    assert (d["j"], d["block"], d["grid"]) == ("11", "512", "512")
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 1024, 11008, 4096, 8192)
    assert (d["j"], d["block"], d["grid"]) == ("11", "256", "256")
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 16, 13, 4096, 8192)
    assert d["kernel"] == "scalar" and d["fallback"] == "1"
    d = _capi.describe_launch("qgemv", "qgemv_wave_r4", 64, 4096, 4096, 8192)
    assert (d["kernel"], d["r"]) == ("wave", "4")


def test_argument_errors_without_launch():
    lib = _capi.load()
    P = 0x1000
    st = lib.cq_int4gemv(b"no_such_variant", P, P, P, P, 4, 128, None)
    assert st == _capi.CQ_ERR_UNKNOWN_VARIANT and "no_such_variant" in _capi.last_error()
    st = lib.cq_int4gemv(b"int4gemv_cdna4", P, P, P, P, 4, 100, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and "128" in _capi.last_error()
    st = lib.cq_int4gemv(b"int4gemv_cdna4", None, P, P, P, 4, 128, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and "null" in _capi.last_error()
    st = lib.cq_int4gemv(b"int4gemv_cdna4", P, P, P, P, 0, 128, None)
    assert st == _capi.CQ_ERR_INVALID_ARG
    st = lib.cq_qgemv(b"qgemv_cdna4", P, P, P, P, 4, 0, None)
    assert st == _capi.CQ_ERR_INVALID_ARG
    st = lib.cq_qgemv(None, P, P, P, P, 4, 4, None)
    assert st == _capi.CQ_ERR_INVALID_ARG
    t = _capi.CqTiming()
    st = lib.cq_native_timing(0, b"int4gemv_cdna4", P, P, P, P, 4, 128, None,
                              -1, 1, 1, None, ctypes.byref(t))
    assert st == _capi.CQ_ERR_INVALID_ARG and "warmup" in _capi.last_error()
    st = lib.cq_pool_timing(0, b"int4gemv_cdna4", None, None, None, None, 1,
                            4, 128, None, 0, 1, None, None)
    assert st == _capi.CQ_ERR_INVALID_ARG
    tot = ctypes.c_double()
    bufs = (ctypes.c_void_p * 2)(0x1000, 0x2008)
    st = lib.cq_read_ceiling(bufs, 2, 4096, P, None, 0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "aligned" in _capi.last_error()
    bufs = (ctypes.c_void_p * 1)(0x1000)
    st = lib.cq_read_ceiling(bufs, 1, 4100, P, None, 0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "multiple of 16" in _capi.last_error()
    st = lib.cq_read_ceiling(bufs, 1, 4096, P, None, 0, 0, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG
    st = lib.cq_read_ceiling(bufs, 1, 4096, None, None, 0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "null" in _capi.last_error()
    st = lib.cq_launch_floor(256, 512, None, None, 0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "null" in _capi.last_error()
    st = lib.cq_launch_floor(256, 512, P, None, 0, 0, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "n_launches" in _capi.last_error()
    for grid, block in ((0, 256), (1 << 31, 256), (256, 0), (256, 1025)):
        st = lib.cq_launch_floor(grid, block, P, None, 0, 1, ctypes.byref(tot))
        assert st == _capi.CQ_ERR_INVALID_ARG and "grid must be" in _capi.last_error()


def test_grouped_argument_errors_without_launch():
    lib = _capi.load()
    P = 0x1000
    probs = (_capi.CqProblem * 3)()
    for i in range(3):
        probs[i].w = probs[i].scale = probs[i].x = probs[i].y = P
        probs[i].n = 8
    st = lib.cq_int4gemv_grouped(b"int4gemv_cdna4", None, 1, 128, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and "NULL" in _capi.last_error()
    st = lib.cq_int4gemv_grouped(b"int4gemv_cdna4", probs, 0, 128, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and "n_problems" in _capi.last_error()
    st = lib.cq_int4gemv_grouped(b"nope", probs, 3, 128, None)
    assert st == _capi.CQ_ERR_UNKNOWN_VARIANT
    st = lib.cq_int4gemv_grouped(b"int4gemv_cdna4", probs, 3, 100, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and "128" in _capi.last_error()
    probs[1].y = None
    st = lib.cq_int4gemv_grouped(b"int4gemv_cdna4", probs, 3, 128, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and _capi.last_error().startswith("problem 1:")
    probs[1].y = P
    probs[2].n = 0
    st = lib.cq_qgemv_grouped(b"qgemv_cdna4", probs, 3, 16, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and _capi.last_error().startswith("problem 2:")



@pytest.mark.parametrize("op,n,k,kernel,cw,j,block", [
    ("gemv_f16", 4096, 4096, "lds", 64, 8, 512),
    ("gemv_f32", 4096, 4096, "lds", 64, 16, 512),
    ("gemv_f16", 4096, 11008, "lds", 64, 22, 512),
    ("gemv_f32", 11008, 4096, "lds", 64, 16, 512),
    ("gemv_f16", 1024, 4096, "lds", 64, 8, 256),   # 512 would leave CUs idle
    ("gemv_f16", 7, 64, "lds", 16, 1, 256),
    ("gemv_f32", 4096, 16384, "scalar", 0, 0, 0),    # x above the LDS limit
    ("gemv_f16", 16, 13, "scalar", 0, 0, 0),         # K % 8 != 0
])
def test_gemv_launch_plans(op, n, k, kernel, cw, j, block):
    d = _capi.describe_launch(op, "gemv_cdna4", n, k, 4096, 8192)
    assert (d["kernel"], int(d["cw"]), int(d["j"])) == (kernel, cw, j)
    if kernel == "lds":
        assert d["fallback"] == "0" and int(d["block"]) == block
        assert int(d["grid"]) == -(-n // ((64 // cw) * (block // 64)))
    else:
        assert d["fallback"] == "1"


def test_gemv_argument_errors_without_launch():
    lib = _capi.load()
    P = 0x1000
    assert lib.cq_gemv(b"gemv_cdna4", 2, P, P, P, 4, 8, None) == _capi.CQ_ERR_INVALID_ARG
    assert "dtype" in _capi.last_error()
    assert lib.cq_gemv(b"nope", 0, P, P, P, 4, 8, None) == _capi.CQ_ERR_UNKNOWN_VARIANT
    assert lib.cq_gemv(b"gemv_cdna4", 0, None, P, P, 4, 8, None) == _capi.CQ_ERR_INVALID_ARG
    assert lib.cq_gemv(b"gemv_cdna4", 1, P, P, P, 4, 0, None) == _capi.CQ_ERR_INVALID_ARG
    # the gemv registry is shared by both dtype ids
    assert _capi.variant_list("gemv_f32", _capi.CQ_LIST_ALL) == \
        _capi.variant_list("gemv_f16", _capi.CQ_LIST_ALL)
    assert _capi.vec_contract_ok("gemv_f32", 0x1000, 0x2000, 12)
    assert not _capi.vec_contract_ok("gemv_f16", 0x1000, 0x2000, 12)
