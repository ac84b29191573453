"""GPU tests of the on-device quantizers (cq_int4_quantize, cq_q8_quantize)
through the C ABI: bit-exact against the oracle's quantizers (the
reference's formula, cudalab/int4gemv_quantize.py:61-114 and
cudalab/qgemv_quantize.py:33-64) in both scale forms (the reference's
`amax / qmax` as torch rounds it on the CPU and on a GPU), on the
reference's shapes and input modes, on crafted ties / near-ties /
subnormal / zero / extreme inputs, on both kernels (vectorized and
element-wise); against the reference's torch formulation run on the same
GPU and on the CPU; and for the NaN/Inf rejection of `quantize_w`."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

import quant_cases as qc

pytestmark = pytest.mark.gpu

MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")
INT4_SHAPES = [(1, 128), (3, 128), (16, 256), (8, 128), (1, 4096), (33, 1024),
               (1024, 4096), (4096, 1024), (4096, 4096), (4099, 4096),
               (11008, 4096), (4096, 11008)]
# The vectorized INT8 kernel holds 1, 2, 3, 4, 6 or 8 chunks of 8 per
# thread: (33, 1000), (1, 4096), (7, 6144), (9, 8192), (4, 12288),
# (4096, 11008) cover each; (3, 20000), (2, 32768), (5, 16392) are longer
# than the 16384 elements a workgroup holds (the rest is re-read);
# (16, 13), (8, 7), (4096, 1): k % 8 != 0, the element-wise kernel.
Q8_SHAPES = [(1, 1), (1, 4096), (4096, 1), (16, 13), (8, 7), (33, 1000),
             (7, 6144), (9, 8192), (4, 12288),
             (1024, 4096), (4096, 4096), (11008, 4096), (4096, 11008),
             (3, 20000), (2, 32768), (5, 16392)]


def _w_cpu(N, K, mode, seed=0):
    from cudalab_amd.operators.gemv import make_w
    return make_w(N, K, torch.float16, device="cpu", seed=seed, mode=mode,
                  large=10.0)


def _eq4(W16: np.ndarray, wp: torch.Tensor, s: torch.Tensor, what, rcp=True):
    owp, os_ = orc.quantize_w4_c(W16, rcp=rcp)
    assert np.array_equal(wp.cpu().numpy(), owp), what
    assert np.array_equal(s.cpu().numpy().view(np.uint16), os_.view(np.uint16)), what


def _eq8(W16: np.ndarray, wq: torch.Tensor, s: torch.Tensor, what, rcp=True):
    owq, os_ = orc.quantize_w8_c(W16, rcp=rcp)
    assert np.array_equal(wq.cpu().numpy(), owq), what
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32)), what


@pytest.fixture(scope="module")
def lib(cuda):
    from cudalab_amd import _capi
    return _capi.load()


@pytest.mark.parametrize("N,K", INT4_SHAPES)
def test_int4_shapes_and_modes(cuda, N, K):
    from cudalab_amd.int4gemv_quantize import quantize_w
    for mode in MODES:
        W = _w_cpu(N, K, mode)
        for sem in ("gpu", "cpu"):
            announce(f"int4 quantize N={N} K={K} mode={mode} semantics={sem}")
            wp, s = quantize_w(W.cuda(), semantics=None if sem == "gpu" else sem)
            torch.cuda.synchronize()
            assert wp.shape == (N, K // 2) and wp.dtype == torch.uint8
            assert s.shape == (N, K // 128) and s.dtype == torch.float16
            _eq4(W.numpy(), wp, s, (N, K, mode, sem), rcp=sem == "gpu")


@pytest.mark.parametrize("N,K", Q8_SHAPES)
def test_q8_shapes_and_modes(cuda, N, K):
    from cudalab_amd.qgemv_quantize import quantize_w
    for mode in MODES:
        W = _w_cpu(N, K, mode)
        for sem in ("gpu", "cpu"):
            announce(f"int8 quantize N={N} K={K} mode={mode} semantics={sem}")
            wq, s = quantize_w(W.cuda(), semantics=None if sem == "gpu" else sem)
            torch.cuda.synchronize()
            assert wq.shape == (N, K) and wq.dtype == torch.int8
            assert s.shape == (N,) and s.dtype == torch.float32
            _eq8(W.numpy(), wq, s, (N, K, mode, sem), rcp=sem == "gpu")


def _offset_copy(t: torch.Tensor, byte_offset: int) -> torch.Tensor:
    """Same values, base pointer `byte_offset` bytes past an aligned one."""
    el = t.element_size()
    flat = torch.zeros(t.numel() + 64 // el, dtype=t.dtype, device=t.device)
    v = flat[byte_offset // el: byte_offset // el + t.numel()].view_as(t)
    v.copy_(t)
    return v


def _raw4(lib, W, wp_off=0, mode=1):
    """cq_int4_quantize on W into an output placed wp_off bytes past an
    aligned base; returns (packed, scale, took_vectorized_kernel)."""
    N, K = W.shape
    buf = torch.zeros(N * K // 2 + 64, dtype=torch.uint8, device=W.device)
    wp = buf[wp_off: wp_off + N * K // 2].view(N, K // 2)
    s = torch.empty(N, K // 128, dtype=torch.float16, device=W.device)
    fast = lib.cq_quantize_vectorized(0, W.data_ptr(), wp.data_ptr(), N, K)
    st = lib.cq_int4_quantize(W.data_ptr(), wp.data_ptr(), s.data_ptr(), N, K,
                              mode, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    return wp, s, fast


def _raw8(lib, W, wq_off=0, mode=1):
    N, K = W.shape
    buf = torch.zeros(N * K + 64, dtype=torch.int8, device=W.device)
    wq = buf[wq_off: wq_off + N * K].view(N, K)
    s = torch.empty(N, dtype=torch.float32, device=W.device)
    fast = lib.cq_quantize_vectorized(1, W.data_ptr(), wq.data_ptr(), N, K)
    st = lib.cq_q8_quantize(W.data_ptr(), wq.data_ptr(), s.data_ptr(), N, K,
                            mode, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    return wq, s, fast


@pytest.mark.parametrize("mode", [0, 1], ids=["div", "rcp"])
@pytest.mark.parametrize("case", sorted(qc.all_cases(7)))
def test_int4_crafted_both_kernels(lib, case, mode):
    W16 = qc.all_cases(7)[case]
    W = torch.from_numpy(W16).cuda()
    announce(f"int4 quantize crafted {case} mode={mode} vectorized")
    wp, s, fast = _raw4(lib, W, 0, mode)
    assert fast == 1
    _eq4(W16, wp, s, case, rcp=mode == 1)
    for w_off, o_off in ((2, 0), (0, 1), (6, 3)):
        announce(f"int4 quantize crafted {case} mode={mode} element-wise w+{w_off} out+{o_off}")
        Wm = _offset_copy(W, w_off) if w_off else W
        wp2, s2, fast2 = _raw4(lib, Wm, o_off, mode)
        assert fast2 == 0
        assert torch.equal(wp2, wp) and torch.equal(s2.view(torch.int16), s.view(torch.int16))


@pytest.mark.parametrize("mode", [0, 1], ids=["div", "rcp"])
@pytest.mark.parametrize("case", sorted(qc.all_cases(127)))
def test_q8_crafted_both_kernels(lib, case, mode):
    W16 = qc.all_cases(127)[case]
    W = torch.from_numpy(W16).cuda()
    announce(f"int8 quantize crafted {case} mode={mode} vectorized")
    wq, s, fast = _raw8(lib, W, 0, mode)
    assert fast == 1
    _eq8(W16, wq, s, case, rcp=mode == 1)
    for w_off, o_off in ((2, 0), (0, 4), (8, 1)):
        announce(f"int8 quantize crafted {case} mode={mode} element-wise w+{w_off} out+{o_off}")
        Wm = _offset_copy(W, w_off) if w_off else W
        wq2, s2, fast2 = _raw8(lib, Wm, o_off, mode)
        assert fast2 == 0
        assert torch.equal(wq2, wq) and torch.equal(s2.view(torch.int32), s.view(torch.int32))


@pytest.mark.parametrize("N,K", [(4096, 4096), (11008, 4096)])
def test_torch_formulation_agrees_on_each_device(cuda, N, K):
    """The reference's torch formulation run on this GPU gives the bytes of
    the HIP quantizers' default (GPU) form; run on the CPU, those of the
    "cpu" form; and the two forms do differ on these weights."""
    from cudalab_amd import int4gemv_quantize as q4, qgemv_quantize as q8
    Wh = _w_cpu(N, K, "normal", seed=3)
    W = Wh.cuda()
    announce(f"quantize torch-vs-hip N={N} K={K}")

    def same(a, b):
        return torch.equal(a[0].cpu(), b[0].cpu()) and torch.equal(
            a[1].cpu().view(torch.int16 if a[1].dtype == torch.float16 else torch.int32),
            b[1].cpu().view(torch.int16 if b[1].dtype == torch.float16 else torch.int32))

    for q in (q4, q8):
        gpu_hip, gpu_torch = q.quantize_w(W), q.quantize_w_torch(W)
        assert same(gpu_hip, gpu_torch), q.__name__
        cpu_hip, cpu_torch = q.quantize_w(W, semantics="cpu"), q.quantize_w_torch(Wh)
        assert same(cpu_hip, cpu_torch), q.__name__
        assert not torch.equal(gpu_hip[0], cpu_hip[0]), q.__name__


def test_nonfinite_rejected_and_located(cuda):
    """NaN or Inf anywhere: quantize_w raises the reference's ValueError;
    the raw kernel marks exactly the groups (INT4) / rows (INT8) holding
    one with a non-finite scale."""
    from cudalab_amd import ext, int4gemv_quantize as q4, qgemv_quantize as q8
    N, K = 64, 1024
    for bad in (float("nan"), float("inf"), float("-inf")):
        W = _w_cpu(N, K, "normal", seed=5)
        rng = np.random.default_rng(1)
        pos = [(int(rng.integers(0, N)), int(rng.integers(0, K))) for _ in range(5)]
        for (r, c) in pos:
            W[r, c] = bad
        Wc = W.cuda()
        announce(f"quantize non-finite {bad}")
        with pytest.raises(ValueError, match="finite"):
            q4.quantize_w(Wc)
        with pytest.raises(ValueError, match="finite"):
            q8.quantize_w(Wc)
        _, s4 = ext.quantize_int4(Wc)
        _, s8 = ext.quantize_q8(Wc)
        want4 = np.zeros((N, K // 128), dtype=bool)
        want8 = np.zeros(N, dtype=bool)
        for (r, c) in pos:
            want4[r, c // 128] = True
            want8[r] = True
        assert np.array_equal(~torch.isfinite(s4).cpu().numpy(), want4)
        assert np.array_equal(~torch.isfinite(s8).cpu().numpy(), want8)


def test_metadata_errors_and_empty(cuda):
    from cudalab_amd import int4gemv_quantize as q4, qgemv_quantize as q8
    with pytest.raises(ValueError, match="divisible by 128"):
        q4.quantize_w(torch.zeros(2, 200, dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError, match="fp16"):
        q4.quantize_w(torch.zeros(2, 256, device="cuda"))
    with pytest.raises(ValueError, match="contiguous"):
        q8.quantize_w(torch.zeros(256, 2, dtype=torch.float16, device="cuda").t())
    wp, s = q4.quantize_w(torch.zeros(0, 256, dtype=torch.float16, device="cuda"))
    assert wp.shape == (0, 128) and s.shape == (0, 2)
    wq, s = q8.quantize_w(torch.zeros(0, 7, dtype=torch.float16, device="cuda"))
    assert wq.shape == (0, 7) and s.shape == (0,)


def test_side_stream_and_repeat(cuda):
    """Launches go on the current stream; repeated calls are identical."""
    from cudalab_amd import ext
    W = _w_cpu(512, 4096, "normal", seed=8).cuda()
    ref = ext.quantize_int4(W)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        outs = [ext.quantize_int4(W) for _ in range(3)]
    torch.cuda.synchronize()
    for wp, s in outs:
        assert torch.equal(wp, ref[0]) and torch.equal(s.view(torch.int16), ref[1].view(torch.int16))


def test_quantized_weights_feed_the_gemv(ext4, ext8):
    """Device-quantized weights through both GEMVs stay within the
    accumulation bound against the oracle."""
    from cudalab_amd import ext
    W = _w_cpu(1024, 4096, "normal", seed=9).cuda()
    x = torch.randn(4096, generator=torch.Generator().manual_seed(2)).half().cuda()
    wp, s = ext.quantize_int4(W)
    y = ext4.forward("int4gemv_cdna4", wp, s, x)
    ex, S = orc.exact_w4(wp.cpu().numpy(), s.cpu().numpy(), x.cpu().numpy())
    assert orc.arith_ratio(y.cpu().numpy(), ex, S, 4096).max() <= 1.0
    wq, s8 = ext.quantize_q8(W)
    y8 = ext8.forward("qgemv_cdna4", wq, s8, x)
    ex, S = orc.exact_w8(wq.cpu().numpy(), s8.cpu().numpy(), x.cpu().numpy())
    assert orc.arith_ratio(y8.cpu().numpy(), ex, S, 4096).max() <= 1.0
