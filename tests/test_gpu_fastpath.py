"""The eager fast path on the GPU (csrc/cq_pyfast.cpp): forward and
forward_into through the cached prepared launch give bit-identical outputs
to the checked path's direct launch, for every variant of the three
operators; the cache holds one entry per operand set and reuses it; a full
cache is cleared and refilled without changing results; calls the fast path
declines (an output overlapping an input) still raise the checked path's
message; and a prepared launch enqueues on the current stream, including a
side stream and a graph capture."""
from __future__ import annotations

import ctypes

import pytest
import torch

from cudalab_amd import _capi
from cudalab_amd import ext as E
from conftest import announce

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def extg(cuda):
    from cudalab_amd.build import build
    return build("gemv")


def _int4(N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    W = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device="cuda", generator=g)
    s = (torch.rand(N, K // 128, device="cuda", generator=g) * 0.02 + 1e-3).half()
    x = torch.randn(K, device="cuda", generator=g).half()
    return W, s, x


def _q8(N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    W = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    s = torch.rand(N, device="cuda", generator=g) * 0.01 + 1e-4
    x = torch.randn(K, device="cuda", generator=g).half()
    return W, s, x


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.float16 else t.view(torch.int32)


def _direct(e, v, W, s, x):
    """The checked path's launch (ctypes, no cache)."""
    out = torch.full((W.size(0),), float("nan"), dtype=torch.float16, device="cuda")
    e._launch(v, W, s, x, out)
    return out


@pytest.mark.parametrize("op,N,K", [("int4gemv", 4096, 4096), ("int4gemv", 300, 1280),
                                    ("int4gemv", 64, 20480), ("qgemv", 4096, 4096),
                                    ("qgemv", 300, 1040), ("qgemv", 7, 16400)])
def test_fast_path_bit_identical_to_direct_launch(ext4, ext8, op, N, K):
    e = ext4 if op == "int4gemv" else ext8
    W, s, x = (_int4 if op == "int4gemv" else _q8)(N, K, seed=N + K)
    for v in e.all_variants():
        announce(f"fast path {op} {v} {N}x{K}")
        want = _direct(e, v, W, s, x)
        out = torch.full_like(want, float("nan"))
        assert e._fast.into(v, W, s, x, out) is True
        y = e._fast.forward(v, W, s, x)
        assert y is not None
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(want)), v
        assert torch.equal(_bits(y), _bits(want)), v


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["f16", "f32"])
def test_gemv_fast_path_bit_identical(extg, dtype):
    g = torch.Generator(device="cuda").manual_seed(5)
    for N, K in ((4096, 4096), (33, 1000), (3, 16376)):
        W = torch.randn(N, K, device="cuda", generator=g).to(dtype)
        x = torch.randn(K, device="cuda", generator=g).to(dtype)
        for v in extg.all_variants():
            announce(f"fast path gemv {v} {dtype} {N}x{K}")
            want = torch.empty(N, dtype=dtype, device="cuda")
            extg._launch2(v, W, x, want)
            out = torch.empty_like(want)
            assert extg._fast.gemv_into(v, W, x, out) is True
            y = extg._fast.gemv_forward(v, W, x)
            torch.cuda.synchronize()
            assert torch.equal(_bits(out), _bits(want)), v
            assert torch.equal(_bits(y), _bits(want)), v


def test_cache_one_entry_per_operand_set(ext4):
    fast = ext4._fast
    fast.clear()
    sets = [_int4(1024, 4096, seed=i) for i in range(3)]
    outs = [torch.empty(1024, dtype=torch.float16, device="cuda") for _ in sets]
    announce("fast path cache entries")
    for _ in range(5):
        for (W, s, x), o in zip(sets, outs):
            ext4.forward_into("int4gemv_cdna4", W, s, x, o)
    assert fast.cached() == 3
    for (W, s, x), o in zip(sets, outs):
        assert torch.equal(_bits(o), _bits(_direct(ext4, "int4gemv_cdna4", W, s, x)))
    ext4.forward_into("int4gemv_lds_r1", *sets[0], outs[0])
    assert fast.cached() == 4
    assert torch.equal(_bits(outs[0]), _bits(_direct(ext4, "int4gemv_lds_r1", *sets[0])))


def test_full_cache_is_cleared_and_refilled(ext4):
    names = ext4.all_variants() + sorted(ext4.aliases())
    small = _capi.fast_module().Launcher(0, names, _capi.entry_address("cq_prepare"),
                                         _capi.entry_address("cq_launch_prepared"),
                                         _capi.entry_address("cq_last_error"), 2)
    sets = [_int4(512, 2048, seed=10 + i) for i in range(5)]
    announce("fast path capacity 2")
    for rep in range(2):
        for W, s, x in sets:
            y = small.forward("int4gemv_cdna4", W, s, x)
            torch.cuda.synchronize()
            assert torch.equal(_bits(y), _bits(_direct(ext4, "int4gemv_cdna4", W, s, x)))
            assert 1 <= small.cached() <= 2


def test_overlapping_output_is_declined_and_raises(ext4):
    W, s, x = _int4(256, 1024, seed=3)
    out = x[:256]                 # the output aliases x
    announce("fast path overlap declined")
    assert ext4._fast.into("int4gemv_cdna4", W, s, x, out) is False
    with pytest.raises(RuntimeError, match="overlaps"):
        ext4.forward_into("int4gemv_cdna4", W, s, x, out)


def test_prepared_launch_follows_the_current_stream(ext4):
    W, s, x = _int4(4096, 4096, seed=4)
    want = _direct(ext4, "int4gemv_cdna4", W, s, x)
    side = torch.cuda.Stream()
    out = torch.full_like(want, float("nan"))
    announce("fast path on a side stream")
    peek = torch.cuda.Stream()
    host = torch.empty(out.shape, dtype=out.dtype, pin_memory=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        torch.cuda._sleep(100_000_000)            # hold the side stream busy (tens of ms)
        ext4.forward_into("int4gemv_cdna4", W, s, x, out)
        done = torch.cuda.Event()
        done.record(side)
    # a third stream reads `out` while the side stream still waits: the
    # launch queued behind the wait has not run, so `out` still holds NaN
    with torch.cuda.stream(peek):
        host.copy_(out, non_blocking=True)
        peeked = torch.cuda.Event()
        peeked.record(peek)
    peeked.synchronize()
    assert not done.query(), "the side stream's wait ended before the peek"
    assert torch.isnan(host.float()).all()
    done.synchronize()
    assert torch.equal(_bits(out), _bits(want))
    announce("fast path under graph capture")
    g = torch.cuda.CUDAGraph()
    cap = torch.full_like(want, float("nan"))
    ext4.forward_into("int4gemv_cdna4", W, s, x, cap)  # warm the cache outside capture
    torch.cuda.synchronize()
    cap.fill_(float("nan"))
    with torch.cuda.graph(g, stream=side):
        ext4.forward_into("int4gemv_cdna4", W, s, x, cap)
    for _ in range(3):
        cap.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(cap), _bits(want))


def test_prepared_record_c_api(ext4):
    """cq_prepare + cq_launch_prepared directly: the same output as
    cq_int4gemv; a zeroed or damaged record is refused."""
    lib = _capi.load()
    W, s, x = _int4(1024, 4096, seed=6)
    want = _direct(ext4, "int4gemv_cdna4", W, s, x)
    out = torch.full_like(want, float("nan"))
    rec = _capi.CqPrepared()
    st = lib.cq_prepare(_capi.CQ_OP_INT4GEMV, b"int4gemv_cdna4", W.data_ptr(), s.data_ptr(),
                        x.data_ptr(), out.data_ptr(), 1024, 4096, ctypes.byref(rec))
    assert st == _capi.CQ_OK, _capi.last_error()
    stream = torch.cuda.current_stream().cuda_stream
    announce("cq_launch_prepared")
    assert lib.cq_launch_prepared(ctypes.addressof(rec), stream) == _capi.CQ_OK
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(want))
    bad = _capi.CqPrepared()
    assert lib.cq_launch_prepared(ctypes.addressof(bad), stream) == _capi.CQ_ERR_INVALID_ARG
    rec.opaque[5] ^= 1
    assert lib.cq_launch_prepared(ctypes.addressof(rec), stream) == _capi.CQ_ERR_INVALID_ARG
    assert "cq_prepare" in _capi.last_error()
    assert E.FAST_CACHE_ENTRIES >= 1024


@pytest.mark.parametrize("op", ["int4gemv", "qgemv"])
def test_grouped_fast_path_matches_single_calls(ext4, ext8, op):
    """forward_grouped through the fast path: every output bit-identical to
    forward_into of its problem; a mixed-K group is declined and raises the
    checked path's message; an iterator still works (checked path)."""
    e, make = (ext4, _int4) if op == "int4gemv" else (ext8, _q8)
    v = "int4gemv_cdna4" if op == "int4gemv" else "qgemv_cdna4"
    probs = [make(N, 4096, seed=40 + N) for N in (4096, 1024, 1024, 300)]
    outs = [torch.full((W.size(0),), float("nan"), dtype=torch.float16, device="cuda")
            for W, _, _ in probs]
    announce(f"grouped fast path {op}")
    assert e._fast.grouped(v, [(W, s, x, o) for (W, s, x), o in zip(probs, outs)]) is True
    for (W, s, x), o in zip(probs, outs):
        want = torch.empty_like(o)
        e._launch(v, W, s, x, want)
        torch.cuda.synchronize()
        assert torch.equal(_bits(o), _bits(want))
    other = make(64, 2048, seed=9)
    mixed = [(*probs[0], outs[0]), (*other, torch.empty(64, dtype=torch.float16, device="cuda"))]
    assert e._fast.grouped(v, mixed) is False
    with pytest.raises(RuntimeError, match="相同的 K"):
        e.forward_grouped(v, mixed)
    outs2 = [torch.empty_like(o) for o in outs]
    e.forward_grouped(v, ((W, s, x, o) for (W, s, x), o in zip(probs, outs2)))
    torch.cuda.synchronize()
    for o, o2 in zip(outs, outs2):
        assert torch.equal(_bits(o), _bits(o2))
