"""GPU tests: the GEMV incumbents are deterministic.  The same inputs give
bit-identical outputs launch after launch, with other launches of other
shapes in between, on the default stream and on a side stream, for the
untiled and K-tiled kernels of the INT4, INT8 and FP16/FP32 operators and
for the grouped entry point.  The kernels have no atomics and a fixed
per-row summation order; these tests pin that property."""
from __future__ import annotations

import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

# untiled (one and two rows per lane), K-tiled, and a short row
SHAPES = [(4096, 4096), (11008, 4096), (4096, 28672), (300, 1280)]
REPEATS = 5


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16 if t.dtype == torch.float16 else torch.int32).clone()


def _repeat(run, out: torch.Tensor, other) -> None:
    """Run `run()` REPEATS times, alternating the default stream and a side
    stream, with `other()` (a launch of another shape) before each, and
    check every output against the first."""
    run()
    torch.cuda.synchronize()
    want = _bits(out)
    side = torch.cuda.Stream()
    for i in range(REPEATS):
        other()
        out.zero_()
        if i % 2:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                run()
            torch.cuda.current_stream().wait_stream(side)
        else:
            run()
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), want), f"repeat {i} differs"


@pytest.mark.parametrize("N,K", SHAPES)
def test_int4_repeats_bit_identically(ext4, N, K):
    from cudalab_amd.operators.int4gemv import device_random_set
    announce(f"determinism int4gemv {N}x{K}")
    W, s, x, y = device_random_set(N, K, 31)
    Wo, so, xo, yo = device_random_set(512, 2048, 33)
    _repeat(lambda: ext4.forward_into("int4gemv_cdna4", W, s, x, y), y,
            lambda: ext4.forward_into("int4gemv_cdna4", Wo, so, xo, yo))


@pytest.mark.parametrize("N,K", SHAPES)
def test_int8_repeats_bit_identically(ext8, N, K):
    from cudalab_amd.operators.qgemv import device_random_set
    announce(f"determinism qgemv {N}x{K}")
    W, s, x, y = device_random_set(N, K, 41)
    Wo, so, xo, yo = device_random_set(512, 2048, 43)
    _repeat(lambda: ext8.forward_into("qgemv_cdna4", W, s, x, y), y,
            lambda: ext8.forward_into("qgemv_cdna4", Wo, so, xo, yo))


@pytest.mark.parametrize("N,K", [(4096, 4096), (4096, 40960), (300, 1280)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_fp_gemv_repeats_bit_identically(cuda, N, K, dtype):
    from cudalab_amd.build import build
    from cudalab_amd.operators.gemv import device_random_set
    ext = build("gemv")
    announce(f"determinism gemv {N}x{K} {dtype}")
    W, x, y = device_random_set(N, K, 51, dtype=dtype)
    Wo, xo, yo = device_random_set(512, 2048, 53, dtype=dtype)
    _repeat(lambda: ext.forward_into("gemv_cdna4", W, x, y), y,
            lambda: ext.forward_into("gemv_cdna4", Wo, xo, yo))


def test_grouped_repeats_bit_identically(ext4, ext8):
    """Three problems of mixed row counts in one grouped call, repeated: each
    output stays bit-identical (and equal to its single forward_into)."""
    from cudalab_amd.operators import int4gemv as o4
    from cudalab_amd.operators import qgemv as o8
    for ext, mod, variant in ((ext4, o4, "int4gemv_cdna4"), (ext8, o8, "qgemv_cdna4")):
        announce(f"determinism grouped {variant}")
        probs = [mod.device_random_set(n, 4096, 61 + n) for n in (4096, 1024, 11008)]
        outs = [p[3] for p in probs]
        ext.forward_grouped(variant, probs)
        torch.cuda.synchronize()
        want = [_bits(o) for o in outs]
        for (W, s, x, o), w in zip(probs, want):
            single = torch.empty_like(o)
            ext.forward_into(variant, W, s, x, single)
            torch.cuda.synchronize()
            assert torch.equal(_bits(single), w)
        for i in range(REPEATS):
            for o in outs:
                o.zero_()
            ext.forward_grouped(variant, probs)
            torch.cuda.synchronize()
            for o, w in zip(outs, want):
                assert torch.equal(_bits(o), w), f"{variant} repeat {i} differs"
