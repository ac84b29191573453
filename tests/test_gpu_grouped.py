"""GPU tests of the grouped GEMV entry points (cq_int4gemv_grouped,
cq_qgemv_grouped): every output of a grouped call is bit-identical to a
single forward_into of the same variant on the same problem, for groups
of one to nine problems (two launches past eight), mixed row counts,
batches where one problem misses the vector contract, and rows longer than
the untiled kernels take; and within the reference's accumulation bound
against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _int4_problem(N, K, seed):
    from cudalab_amd.operators.int4gemv import make_w4, make_x4
    wp, s, _ = make_w4(N, K, seed=seed, mode="normal")
    x = make_x4(K, seed=seed + 1, mode="normal")
    return wp, s, x


def _q8_problem(N, K, seed):
    from cudalab_amd.operators.qgemv import make_w_q, make_x_q
    wq, s, _ = make_w_q(N, K, seed=seed, mode="normal")
    x = make_x_q(K, seed=seed + 1, mode="normal")
    return wq, s, x


def _misalign_w(W):
    """Same values, base pointer 2 bytes past a 16-byte boundary."""
    flat = torch.zeros(W.numel() + 64, dtype=W.dtype, device=W.device)
    view = flat[2:2 + W.numel()].view_as(W)
    view.copy_(W)
    return view


def _check(ext, variant, probs):
    outs = [torch.full((p[0].size(0),), float("nan"), dtype=torch.float16,
                       device="cuda") for p in probs]
    ext.forward_grouped(variant, [(W, s, x, o) for (W, s, x), o in zip(probs, outs)])
    torch.cuda.synchronize()
    for i, ((W, s, x), o) in enumerate(zip(probs, outs)):
        ref = torch.empty_like(o)
        ext.forward_into(variant, W, s, x, ref)
        torch.cuda.synchronize()
        assert torch.equal(o, ref), (variant, i)
    return outs


INT4_GROUPS = {
    "qkv": [(4096, 4096)] * 3,
    "gate_up": [(11008, 4096)] * 2,
    "mixed": [(1, 4096), (33, 4096), (4099, 4096), (300, 4096), (64, 4096)],
    "nine": [(128 + 16 * i, 1024) for i in range(9)],
    "one": [(4096, 11008)],
}


@pytest.mark.parametrize("group", sorted(INT4_GROUPS))
def test_int4_grouped_bit_identical(ext4, group):
    shapes = INT4_GROUPS[group]
    probs = [_int4_problem(N, K, seed=11 + i) for i, (N, K) in enumerate(shapes)]
    for v in ("int4gemv_cdna4", "int4gemv_lds_r1", "int4gemv_lds_r2",
              "int4gemv_wave_r2", "int4gemv_baseline"):
        announce(f"int4 grouped {group} {v}")
        outs = _check(ext4, v, probs)
    K = shapes[0][1]
    for (W, s, x), y in zip(probs, outs):
        ex, S = orc.exact_w4(W.cpu().numpy(), s.cpu().numpy(), x.cpu().numpy())
        assert orc.arith_ratio(y.cpu().numpy(), ex, S, K).max() <= 1.0


def test_int4_grouped_with_misaligned_problem(ext4):
    """A batch holding a problem that misses the vector contract is launched
    problem by problem: the misaligned one on the scalar kernel (bit-identical
    to the baseline), the others as single CDNA4 launches."""
    probs = [_int4_problem(N, 4096, seed=31 + i) for i, N in enumerate((512, 777, 256))]
    W, s, x = probs[1]
    probs[1] = (_misalign_w(W), s, x)
    outs = _check(ext4, "int4gemv_cdna4", probs)
    base = ext4.forward("int4gemv_baseline", *probs[1])
    assert torch.equal(outs[1], base)


Q8_GROUPS = {
    "qkv": [(4096, 4096)] * 3,
    "mixed": [(1, 4096), (1001, 4096), (17, 4096)],
    "nine": [(64 + 8 * i, 1024) for i in range(9)],
}


@pytest.mark.parametrize("group", sorted(Q8_GROUPS))
def test_q8_grouped_bit_identical(ext8, group):
    shapes = Q8_GROUPS[group]
    probs = [_q8_problem(N, K, seed=41 + i) for i, (N, K) in enumerate(shapes)]
    for v in ("qgemv_cdna4", "qgemv_lds_r2", "qgemv_wave_r1", "qgemv_baseline"):
        announce(f"q8 grouped {group} {v}")
        outs = _check(ext8, v, probs)
    K = shapes[0][1]
    for (W, s, x), y in zip(probs, outs):
        ex, S = orc.exact_w8(W.cpu().numpy(), s.cpu().numpy(), x.cpu().numpy())
        assert orc.arith_ratio(y.cpu().numpy(), ex, S, K).max() <= 1.0


def test_q8_grouped_odd_k_falls_back(ext8):
    """K % 16 != 0 misses the vector contract for every problem: the batch
    runs problem by problem on the scalar kernel."""
    probs = [_q8_problem(N, 13, seed=51 + i) for i, N in enumerate((16, 9))]
    outs = _check(ext8, "qgemv_cdna4", probs)
    for (W, s, x), y in zip(probs, outs):
        assert torch.equal(y, ext8.forward("qgemv_baseline", W, s, x))


def test_grouped_long_k_runs_problem_by_problem(ext4, ext8):
    """K above the untiled kernels' limit (16384): a grouped call launches
    each problem on its own K-tiled kernel, bit-identical to single calls,
    on both sides of the tiled plans' 3072-row boundary (one row per wave
    up to 3072 rows, two above) and for a few-row problem."""
    probs = [_int4_problem(N, 28672, seed=61 + i) for i, N in enumerate((3072, 3073, 5))]
    outs = {}
    for v in ("int4gemv_cdna4", "int4gemv_lds_r1", "int4gemv_lds_r2"):
        announce(f"int4 grouped long-k {v}")
        outs[v] = _check(ext4, v, probs)
    # one or two rows per wave, 7- or 2-chunk tiles: the same lane order,
    # so the same bits
    for v, o in outs.items():
        for a, b in zip(o, outs["int4gemv_lds_r1"]):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), v
    probs8 = [_q8_problem(N, 20480, seed=71 + i) for i, N in enumerate((3072, 3073, 7))]
    outs8 = {}
    for v in ("qgemv_cdna4", "qgemv_lds_r1", "qgemv_lds_r2"):
        announce(f"q8 grouped long-k {v}")
        outs8[v] = _check(ext8, v, probs8)
    for v, o in outs8.items():
        for a, b in zip(o, outs8["qgemv_lds_r1"]):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), v


def test_grouped_rejects_dependent_problems(ext4, ext8):
    """The problems of one grouped launch run at the same time, so one
    problem's output may not be another's input or output (that chain needs
    two calls).  Shared inputs stay allowed: q/k/v read one x.  Nothing is
    launched for a rejected call: the outputs keep their contents."""
    announce("grouped overlap rejection int4/int8")
    wp0, s0, x = _int4_problem(256, 1024, seed=61)
    wp1, s1, x1 = _int4_problem(1024, 1024, seed=62)
    y0 = torch.zeros(256, dtype=torch.float16, device="cuda")
    y1 = torch.zeros(1024, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="problem 1: output y overlaps x of problem 0"):
        ext4.forward_grouped("int4gemv_cdna4", [(wp0, s0, x, y0), (wp1, s1, x1, x)])
    with pytest.raises(RuntimeError, match="overlaps"):
        ext4.forward_grouped("int4gemv_cdna4", [(wp0, s0, x, y1[:256]), (wp1, s1, x, y1)])
    with pytest.raises(RuntimeError, match="overlaps an input"):
        ext4.forward_into("int4gemv_cdna4", wp1, s1, x, x)
    torch.cuda.synchronize()
    assert not y0.any() and not y1.any()
    # the same two problems with separate outputs and a shared x are fine
    _check(ext4, "int4gemv_cdna4", [(wp0, s0, x), (wp1, s1, x)])
    wq, sq, xq = _q8_problem(512, 512, seed=63)
    with pytest.raises(RuntimeError, match="overlaps"):
        ext8.forward_grouped("qgemv_cdna4", [(wq, sq, xq, xq), (wq, sq, xq, torch.empty(512, dtype=torch.float16, device="cuda"))])
