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
    # up to 3 chunks per lane: one row per lane while one row per wave keeps
    # the grid resident (n <= 32 waves x 256 CUs), 512 threads when their
    # workgroups fill the CUs in whole rounds (or 8+ rounds)
    (4096, 4096, "lds", 64, 2, 1, 512),      # 512 workgroups: whole rounds
    (8192, 4096, "lds", 64, 2, 1, 512),      # 8192 rows: still resident
    (6144, 4096, "lds", 64, 2, 1, 512),      # 768 workgroups: whole rounds
    (3000, 4096, "lds", 64, 2, 1, 256),      # 375 would leave a partial round
    (1024, 4096, "lds", 64, 2, 1, 256),
    # past 8192 rows one row per wave would run a second round of waves: two
    # rows per lane, on 256-thread workgroups
    (11008, 4096, "lds", 64, 2, 2, 256),
    (8193, 4096, "lds", 64, 2, 2, 256),
    (27648, 5120, "lds", 64, 3, 2, 256),
    # rows of at most 32 chunks (several rows per wave): two rows per lane
    (4096, 1024, "lds", 32, 1, 2, 256),
    (1, 128, "lds", 16, 1, 2, 256),
    (4096, 11008, "lds", 64, 6, 1, 512),
    (5, 16384, "lds", 64, 8, 1, 256),
    # 4+ chunks per lane (k >= 8192): one row per lane at any n
    (8192, 8192, "lds", 64, 4, 1, 512),
    (57344, 8192, "lds", 64, 4, 1, 512),
    (4096, 6144, "lds", 64, 3, 1, 512),
    (5120, 5120, "lds", 64, 3, 1, 256),      # 640: 2.5 rounds
    (5120, 13824, "lds", 64, 7, 1, 256),
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
    # the wave variants hold x in registers: beyond 16384 they fall back
    d = _capi.describe_launch("int4gemv", "int4gemv_wave_r1", 8, 16512, 4096, 8192)
    assert d["kernel"] == "scalar" and d["fallback"] == "1" and "k above" in d["why"]
    d = _capi.describe_launch("int4gemv", "int4gemv_baseline", 8, 4096, 4096, 8192)
    assert d["kernel"] == "scalar" and d["fallback"] == "0"
    d = _capi.describe_launch("int4gemv", "int4gemv_rowtile4_hx", 8, 4096, 4096, 8192)
    assert d["variant"] == "int4gemv_cdna4" and d["kernel"] == "lds"
    # weights of 4 GiB or more would overflow the untiled kernels' 32-bit
    # offsets: the tiled kernel (64-bit row bases) takes them
    d = _capi.describe_launch("int4gemv", "int4gemv_cdna4", 1 << 20, 8192, 4096, 8192)
    assert d["kernel"] == "tiled" and d["fallback"] == "0"
    d = _capi.describe_launch("int4gemv", "int4gemv_cdna4", (1 << 20) - 1, 8192, 4096, 8192)
    assert d["kernel"] == "lds"


@pytest.mark.parametrize("op,variant,n,k,j,r,tile", [
    # k above 16384: the LDS variants run the K-tiled kernel on 256-thread
    # workgroups.  INT4: two rows per wave above n = 3072, with 2-chunk
    # tiles up to 16 chunks per lane and 4-chunk tiles beyond; one row up to
    # 3072 with 7-chunk tiles.  INT8: two rows above 3072 with 4-chunk tiles,
    # one row up to 3072 with 8-chunk tiles.
    ("int4gemv", "int4gemv_cdna4", 8, 16512, 9, 1, 7),
    ("int4gemv", "int4gemv_cdna4", 8192, 28672, 14, 2, 2),
    ("int4gemv", "int4gemv_cdna4", 4096, 32768, 16, 2, 2),
    ("int4gemv", "int4gemv_cdna4", 4096, 32896, 17, 2, 4),
    ("int4gemv", "int4gemv_cdna4", 3073, 28672, 14, 2, 2),
    ("int4gemv", "int4gemv_cdna4", 3072, 28672, 14, 1, 7),
    ("int4gemv", "int4gemv_cdna4", 2047, 28672, 14, 1, 7),
    ("int4gemv", "int4gemv_lds_r2", 100, 20480, 10, 2, 2),     # rows requested
    ("int4gemv", "int4gemv_lds_r1", 8192, 20480, 10, 1, 7),
    ("int4gemv", "int4gemv_cdna4", 2048, 65536, 32, 1, 7),
    ("int4gemv", "int4gemv_cdna4", 16384, 65536, 32, 2, 4),
    ("qgemv", "qgemv_cdna4", 8192, 28672, 28, 2, 4),
    ("qgemv", "qgemv_cdna4", 4096, 28672, 28, 2, 4),
    ("qgemv", "qgemv_cdna4", 2048, 28672, 28, 1, 8),
    ("qgemv", "qgemv_cdna4", 3328, 28672, 28, 2, 4),
    ("qgemv", "qgemv_cdna4", 3, 16400, 17, 1, 8),
    # the *_lds_tiled variants force it at any k
    ("int4gemv", "int4gemv_lds_tiled", 4096, 4096, 2, 2, 2),
    ("int4gemv", "int4gemv_lds_tiled", 1, 128, 1, 1, 7),
    ("qgemv", "qgemv_lds_tiled", 4097, 11008, 11, 2, 4),
])
def test_tiled_plans(op, variant, n, k, j, r, tile):
    d = _capi.describe_launch(op, variant, n, k, 4096, 8192)
    assert d["kernel"] == "tiled" and d["fallback"] == "0"
    assert (int(d["cw"]), int(d["j"]), int(d["r"]), int(d["block"])) == (64, j, r, 256)
    assert int(d["tile"]) == tile
    assert int(d["grid"]) == -(-(-(-n // r)) // 4)


def test_fp16_tiled_plan_reports_its_tile():
    d = _capi.describe_launch("gemv_f16", "gemv_lds_tiled", 4096, 4096, 4096, 8192)
    assert d["kernel"] == "tiled" and d["tile"] == "32"


def test_untiled_plans_report_no_tile():
    for op, variant, k in (("int4gemv", "int4gemv_cdna4", 4096), ("qgemv", "qgemv_cdna4", 4096),
                           ("int4gemv", "int4gemv_baseline", 4096), ("gemv_f16", "gemv_cdna4", 4096)):
        assert _capi.describe_launch(op, variant, 4096, k, 4096, 8192)["tile"] == "0", variant


def test_tiled_keeps_the_fallbacks():
    """The tiled kernel has the same vector contract and 32-bit offsets."""
    d = _capi.describe_launch("int4gemv", "int4gemv_lds_tiled", 8, 4096, 4098, 8192)
    assert d["kernel"] == "scalar" and "alignment" in d["why"]
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 8, 16392, 4096, 8192)   # k % 16
    assert d["kernel"] == "scalar" and "k%16" in d["why"]
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 1 << 14, 1 << 18, 4096, 8192)
    assert d["kernel"] == "tiled"                       # 4 GiB of weights
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 1 << 18, 1 << 14, 4096, 8192)
    assert d["kernel"] == "tiled" and d["r"] == "2"     # 4 GiB, short rows
    d = _capi.describe_launch("gemv_f16", "gemv_cdna4", 1 << 17, 1 << 14, 4096, 8192)
    assert d["kernel"] == "tiled"                       # 4 GiB of fp16 weights
    d = _capi.describe_launch("gemv_f32", "gemv_cdna4", 2, 1 << 30, 4096, 8192)
    assert d["kernel"] == "scalar" and "rows of 4 GiB" in d["why"]
    d = _capi.describe_launch("qgemv", "qgemv_wave_r1", 8, 16400, 4096, 8192)
    assert d["kernel"] == "scalar" and "k above" in d["why"]


@pytest.mark.parametrize("op,variants,step", [
    ("int4gemv", ("int4gemv_cdna4", "int4gemv_lds_r1", "int4gemv_lds_r2",
                  "int4gemv_lds_r4", "int4gemv_wave_r1"), 128),
    ("qgemv", ("qgemv_cdna4", "qgemv_lds_r1", "qgemv_lds_r2", "qgemv_wave_r1"), 16),
])
def test_lds_plans_hold_whole_row_chunks(op, variants, step):
    """The LDS kernels read a lane's chunks col + cw*j for j < J-1 without a
    clamp, which stays inside the row only when J = ceil(nchunks / cw); the
    launch checks it, and every plan must have that form (k up to the
    untiled limit, both operand widths, several row counts)."""
    per_chunk = 32 if op == "int4gemv" else 16
    for variant in variants:
        for k in range(step, 16384 + 1, step):
            nchunks = k // per_chunk
            for n in (1, 4096):
                d = _capi.describe_launch(op, variant, n, k, 4096, 8192)
                if d["kernel"] == "scalar":
                    continue
                cw, j = int(d["cw"]), int(d["j"])
                assert j == -(-nchunks // cw), (variant, n, k, d)


def test_q8_launch_plans():
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 4096, 4096, 4096, 8192)
    assert (d["kernel"], d["cw"], d["j"], d["r"]) == ("lds", "64", "4", "1")
    assert (d["block"], d["grid"]) == ("256", "1024")
    # 8+ chunks per lane and a grid that still covers every CU: 512 threads
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 4096, 11008, 4096, 8192)
    assert (d["j"], d["block"], d["grid"]) == ("11", "512", "512")
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 1024, 11008, 4096, 8192)
    assert (d["j"], d["block"], d["grid"]) == ("11", "256", "256")
    # 640 workgroups of 512 would be 2.5 rounds over the CUs: 256 threads
    d = _capi.describe_launch("qgemv", "qgemv_cdna4", 5120, 13824, 4096, 8192)
    assert (d["j"], d["block"], d["grid"]) == ("14", "256", "1280")
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
                            4, 128, None, 0, 0.0, 0.0, 1, None, None, None)
    assert st == _capi.CQ_ERR_INVALID_ARG
    one = (ctypes.c_void_p * 1)(0x1000)
    for burn, delay, what in ((-1.0, 0.0, "burn_ms"), (float("nan"), 0.0, "burn_ms"),
                              (1e9, 0.0, "burn_ms"), (0.0, -1.0, "delay_us"),
                              (0.0, 2e6, "delay_us"), (0.0, float("inf"), "delay_us")):
        st = lib.cq_pool_timing(0, b"int4gemv_cdna4", one, one, one, one, 1,
                                4, 128, None, 0, burn, delay, 1, None, None, None)
        assert st == _capi.CQ_ERR_INVALID_ARG and what in _capi.last_error()
    tot = ctypes.c_double()
    bufs = (ctypes.c_void_p * 2)(0x1000, 0x2008)
    st = lib.cq_read_ceiling(bufs, 2, 4096, P, None, 0, 0.0, 0.0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "aligned" in _capi.last_error()
    bufs = (ctypes.c_void_p * 1)(0x1000)
    st = lib.cq_read_ceiling(bufs, 1, 4100, P, None, 0, 0.0, 0.0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "multiple of 16" in _capi.last_error()
    st = lib.cq_read_ceiling(bufs, 1, 4096, P, None, 0, 0.0, 0.0, 0, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG
    st = lib.cq_read_ceiling(bufs, 1, 4096, None, None, 0, 0.0, 0.0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "null" in _capi.last_error()
    st = lib.cq_launch_floor(256, 512, None, None, 0, 0.0, 0.0, 1, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "null" in _capi.last_error()
    st = lib.cq_launch_floor(256, 512, P, None, 0, 0.0, 0.0, 0, ctypes.byref(tot))
    assert st == _capi.CQ_ERR_INVALID_ARG and "n_launches" in _capi.last_error()
    for grid, block in ((0, 256), (1 << 31, 256), (256, 0), (256, 1025)):
        st = lib.cq_launch_floor(grid, block, P, None, 0, 0.0, 0.0, 1, ctypes.byref(tot))
        assert st == _capi.CQ_ERR_INVALID_ARG and "grid must be" in _capi.last_error()


def test_timeline_refuses_before_any_launch():
    """cq_int4_timeline's refusals come from host checks alone (fake,
    disjoint device addresses; nothing is launched): null arguments, a set
    whose plan is not the LDS kernel (a misaligned W takes the scalar
    kernel), a stamp buffer too small or overlapping an operand."""
    lib = _capi.load()
    VP1 = ctypes.c_void_p * 1
    w, s, x, y = VP1(0x10000000), VP1(0x20000000), VP1(0x30000000), VP1(0x40000000)
    waves, tpu, tot = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double()

    def call(w, s, x, y, n_sets=1, n=4096, k=4096, launches=2, stamps=0x50000000,
             words=1 << 40):
        return lib.cq_int4_timeline(b"int4gemv_cdna4", w, s, x, y, n_sets, n, k, None,
                                    0, 0.0, 0.0, launches, stamps, words,
                                    ctypes.byref(waves), ctypes.byref(tpu),
                                    ctypes.byref(tot))

    assert call(w, s, x, y, stamps=None) == _capi.CQ_ERR_INVALID_ARG
    assert "null" in _capi.last_error()
    assert call(None, s, x, y) == _capi.CQ_ERR_INVALID_ARG
    assert call(w, s, x, y, launches=0) == _capi.CQ_ERR_INVALID_ARG
    assert "n_launches" in _capi.last_error()
    assert call(VP1(0x10000001), s, x, y) == _capi.CQ_ERR_INVALID_ARG
    assert "covers the LDS kernel" in _capi.last_error()
    # 4096 x 4096: 512 workgroups of 512 threads, 4096 waves, 8 words each
    assert call(w, s, x, y, launches=3, words=3 * 4096 * 8 - 1) == _capi.CQ_ERR_INVALID_ARG
    assert "stamps holds" in _capi.last_error()
    # stamps that share a byte with a set's operand (here: the end of W)
    assert call(w, s, x, y, stamps=0x10000000 + 4096 * 2048 - 8) == _capi.CQ_ERR_INVALID_ARG
    assert "overlap an operand of set 0" in _capi.last_error()
    two = ctypes.c_void_p * 2
    w2 = two(0x10000000, 0x11000000)
    s2 = two(0x20000000, 0x21000000)
    y2 = two(0x40000000, 0x41000000)
    x2 = two(0x30000000, 0x31000008)    # the second x is off 16-byte alignment
    assert call(w2, s2, x2, y2, n_sets=2) == _capi.CQ_ERR_INVALID_ARG
    assert "set 1" in _capi.last_error()


def _prepare(lib, op, variant, w, s, x, y, n, k):
    rec = _capi.CqPrepared()
    for i in range(12):
        rec.opaque[i] = 0xA5A5A5A5A5A5A5A5          # must be overwritten either way
    st = lib.cq_prepare(op, variant, w, s, x, y, n, k, ctypes.byref(rec))
    return st, rec


def test_prepare_checks_like_the_direct_call_and_launches_nothing():
    """cq_prepare runs the direct call's checks with the same statuses and
    messages and zeroes the record on failure; on success it fills a
    deterministic record (same arguments, same bytes).  It makes no GPU
    call, so this runs on the CPU with fake, disjoint device addresses."""
    lib = _capi.load()
    W, S, X, Y = 0x10000000, 0x20000000, 0x30000000, 0x40000000
    for args, status, words in (
            ((0, b"no_such_variant", W, S, X, Y, 8, 128), _capi.CQ_ERR_UNKNOWN_VARIANT, "no_such_variant"),
            ((0, b"int4gemv_cdna4", W, S, X, Y, 8, 100), _capi.CQ_ERR_INVALID_ARG, "128"),
            ((0, b"int4gemv_cdna4", None, S, X, Y, 8, 128), _capi.CQ_ERR_INVALID_ARG, "null"),
            ((0, b"int4gemv_cdna4", W, S, X, X, 8, 128), _capi.CQ_ERR_INVALID_ARG, "overlaps"),
            ((1, b"qgemv_cdna4", W, S, X, Y, 0, 16), _capi.CQ_ERR_INVALID_ARG, "n must be"),
            ((7, b"int4gemv_cdna4", W, S, X, Y, 8, 128), _capi.CQ_ERR_INVALID_ARG, "operator")):
        st, rec = _prepare(lib, *args)
        assert st == status and words in _capi.last_error(), (args, st, _capi.last_error())
        assert list(rec.opaque) == [0] * 12, args
    assert lib.cq_prepare(0, b"int4gemv_cdna4", W, S, X, Y, 8, 128, None) == _capi.CQ_ERR_INVALID_ARG
    st1, r1 = _prepare(lib, 0, b"int4gemv_cdna4", W, S, X, Y, 4096, 4096)
    st2, r2 = _prepare(lib, 0, b"int4gemv_cdna4", W, S, X, Y, 4096, 4096)
    st3, r3 = _prepare(lib, 0, b"int4gemv_lds_r2", W, S, X, Y, 4096, 4096)
    st4, r4 = _prepare(lib, 0, b"int4gemv_rowtile4_hx", W, S, X, Y, 4096, 4096)  # alias
    assert st1 == st2 == st3 == st4 == _capi.CQ_OK, _capi.last_error()
    assert list(r1.opaque) == list(r2.opaque) == list(r4.opaque)
    assert list(r1.opaque) != list(r3.opaque) and any(r1.opaque)
    # the FP16/FP32 GEMV ignores the scale pointer, as cq_gemv does
    sa, ga = _prepare(lib, _capi.CQ_OP_GEMV_F16, b"gemv_cdna4", W, None, X, Y, 64, 64)
    sb, gb = _prepare(lib, _capi.CQ_OP_GEMV_F16, b"gemv_cdna4", W, S, X, Y, 64, 64)
    assert sa == sb == _capi.CQ_OK and list(ga.opaque) == list(gb.opaque)


def test_launch_prepared_refuses_records_prepare_did_not_fill():
    """A zeroed, damaged or null record is refused before any GPU call."""
    lib = _capi.load()
    assert lib.cq_launch_prepared(None, None) == _capi.CQ_ERR_INVALID_ARG
    zero = _capi.CqPrepared()
    assert lib.cq_launch_prepared(ctypes.addressof(zero), None) == _capi.CQ_ERR_INVALID_ARG
    assert "cq_prepare" in _capi.last_error()
    st, rec = _prepare(lib, 0, b"int4gemv_cdna4", 0x10000000, 0x20000000,
                       0x30000000, 0x40000000, 4096, 4096)
    assert st == _capi.CQ_OK
    for word in range(11):                       # every word the seal covers
        bad = _capi.CqPrepared()
        ctypes.memmove(ctypes.byref(bad), ctypes.byref(rec), ctypes.sizeof(rec))
        bad.opaque[word] ^= 1 << (word % 64)
        assert lib.cq_launch_prepared(ctypes.addressof(bad), None) == _capi.CQ_ERR_INVALID_ARG, word


def _disjoint_problems(count, n=8):
    """Problems with non-overlapping fake device addresses (never launched:
    every call below fails its argument checks first)."""
    probs = (_capi.CqProblem * count)()
    for i in range(count):
        probs[i].w = 0x10000000 + i * 0x1000000
        probs[i].scale = probs[i].w + 0x800000
        probs[i].x = 0x70000000 + i * 0x10000
        probs[i].y = 0x80000000 + i * 0x10000
        probs[i].n = n
    return probs


def test_grouped_argument_errors_without_launch():
    lib = _capi.load()
    P = 0x80000000
    probs = _disjoint_problems(3)
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
    probs[1].y = P + 0x10000
    probs[2].n = 0
    st = lib.cq_qgemv_grouped(b"qgemv_cdna4", probs, 3, 16, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and _capi.last_error().startswith("problem 2:")


def test_output_overlap_is_rejected_before_launch():
    """A kernel reads w, scale and x while other workgroups already write y,
    and the problems of a grouped launch run at the same time: an output
    sharing a byte with an input of its own call, or with any operand of
    another problem of the same grouped call, is an argument error.  Inputs
    may be shared (q/k/v read one x).  Nothing here reaches a launch."""
    lib = _capi.load()
    w, sc, x = 0x10000000, 0x20000000, 0x30000000       # k = 128: x is 256 bytes
    for y in (x, x + 254, w + 100, sc):
        st = lib.cq_int4gemv(b"int4gemv_cdna4", w, sc, x, y, 8, 128, None)
        assert st == _capi.CQ_ERR_INVALID_ARG, hex(y)
        assert "overlaps an input" in _capi.last_error()
    st = lib.cq_qgemv(b"qgemv_cdna4", w, sc, x, sc + 31, 8, 16, None)    # scale: 32 B
    assert st == _capi.CQ_ERR_INVALID_ARG and "overlaps" in _capi.last_error()
    st = lib.cq_gemv(b"gemv_cdna4", _capi.CQ_DTYPE_F32, w, x, x + 16 * 4 - 4, 2, 16, None)
    assert st == _capi.CQ_ERR_INVALID_ARG and "overlaps" in _capi.last_error()
    # grouped: y of one problem inside another problem's x, w, scale or y
    cases = [("x", lambda p: setattr(p[1], "y", p[0].x + 2)),
             ("w", lambda p: setattr(p[2], "y", p[0].w + 64)),
             ("scale", lambda p: setattr(p[0], "y", p[2].scale)),
             ("y", lambda p: setattr(p[1], "y", p[2].y + 8))]
    for what, plant in cases:
        probs = _disjoint_problems(3)
        plant(probs)
        st = lib.cq_int4gemv_grouped(b"int4gemv_cdna4", probs, 3, 128, None)
        assert st == _capi.CQ_ERR_INVALID_ARG, what
        msg = _capi.last_error()
        assert f"output y overlaps {what} of problem" in msg, msg
        assert "must be independent" in msg


def test_grouped_overlap_check_scales_and_allows_shared_inputs(monkeypatch):
    """Many problems sharing one x (allowed) with one planted conflict at
    the end: the sorted check finds it without a quadratic scan."""
    lib = _capi.load()
    count = 20000
    probs = _disjoint_problems(count, n=8)
    for i in range(count):
        probs[i].x = 0x70000000                        # shared input
        probs[i].w = 0x100000000 + i * 0x1000
        probs[i].scale = 0x300000000 + i * 0x100
        probs[i].y = 0x500000000 + i * 0x100
    probs[count - 1].y = probs[3].w + 16                # conflict: y inside w of problem 3
    import time
    t0 = time.perf_counter()
    st = lib.cq_int4gemv_grouped(b"int4gemv_cdna4", probs, count, 128, None)
    assert time.perf_counter() - t0 < 5.0
    assert st == _capi.CQ_ERR_INVALID_ARG
    assert _capi.last_error().startswith(f"problem {count - 1}: output y overlaps w of problem 3")



@pytest.mark.parametrize("op,n,k,kernel,cw,j,block", [
    ("gemv_f16", 4096, 4096, "lds", 64, 8, 512),
    ("gemv_f32", 4096, 4096, "lds", 64, 16, 512),
    ("gemv_f16", 4096, 11008, "lds", 64, 22, 512),
    ("gemv_f32", 11008, 4096, "lds", 64, 16, 256),   # 1376 of 512: 5.4 rounds
    ("gemv_f16", 6144, 4096, "lds", 64, 8, 512),     # 768 of 512: 3 whole rounds
    ("gemv_f16", 5120, 13824, "lds", 64, 27, 256),   # 640 of 512: 2.5 rounds
    ("gemv_f16", 1024, 4096, "lds", 64, 8, 256),   # 512 would leave CUs idle
    ("gemv_f16", 7, 64, "lds", 16, 1, 256),
    # x above the 64 KiB stage: the K-tiled kernel, one row per wave
    ("gemv_f32", 4096, 16384, "tiled", 64, 64, 512),
    ("gemv_f16", 8192, 65536, "tiled", 64, 128, 512),
    ("gemv_f16", 300, 40000, "tiled", 64, 79, 256),
    ("gemv_f16", 4096, 32760, "lds", 64, 64, 512),   # the largest x that fits
    ("gemv_f16", 16, 13, "scalar", 0, 0, 0),         # K % 8 != 0
])
def test_gemv_launch_plans(op, n, k, kernel, cw, j, block):
    d = _capi.describe_launch(op, "gemv_cdna4", n, k, 4096, 8192)
    assert (d["kernel"], int(d["cw"]), int(d["j"])) == (kernel, cw, j)
    if kernel in ("lds", "tiled"):
        assert d["fallback"] == "0" and int(d["block"]) == block
        assert int(d["grid"]) == -(-n // ((64 // cw) * (block // 64)))
    else:
        assert d["fallback"] == "1"


def test_gemv_tiled_variant_plans():
    d = _capi.describe_launch("gemv_f16", "gemv_lds_tiled", 4096, 4096, 4096, 8192)
    assert (d["kernel"], d["cw"], d["r"], d["block"]) == ("tiled", "64", "1", "512")
    d = _capi.describe_launch("gemv_f32", "gemv_lds_tiled", 5, 20, 4096, 8192)   # k % 4
    assert d["kernel"] == "tiled" and d["block"] == "256" and d["grid"] == "2"
    d = _capi.describe_launch("gemv_f16", "gemv_lds_tiled", 5, 20, 4096, 8192)   # k % 8
    assert d["kernel"] == "scalar" and d["fallback"] == "1"


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


def test_library_carries_the_source_stamp_of_the_tree():
    from cudalab_amd.build import source_hash
    lib = _capi.load()
    v = lib.cq_version().decode()
    assert v.startswith("cdnaqgemv ") and "(gfx950)" in v
    assert _capi.library_stamp(lib) == source_hash()
    assert len(source_hash()) == 16


def test_stale_library_is_refused(monkeypatch):
    """A library whose stamp differs from the tree's sources does not load."""
    _capi.load()
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setattr(_capi, "source_hash", lambda: "0123456789abcdef")
    with pytest.raises(_capi.StaleLibrary, match="other sources"):
        _capi.load()
