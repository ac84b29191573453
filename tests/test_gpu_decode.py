"""GPU tests of the decode-step driver (cudalab_amd/decode.py): the grouped
step and its HIP-graph replays produce bit-identical outputs to the
one-launch-per-projection step, every replay (with eager work and
synchronizations between replays) matches, and the first projection is
within the reference's accumulation bound against the oracle."""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("op", ["int4gemv", "qgemv"])
def test_decode_modes_bit_identical(cuda, op):
    from cudalab_amd.decode import DecodeModel
    announce(f"decode {op} 2 layers")
    m = DecodeModel(op, layers=2, seed=3)
    m.step_sequential()
    torch.cuda.synchronize()
    ref = m.outputs()
    assert all(torch.isfinite(t).all() for t in ref)
    for L in m.layers:
        for t in L.out.values():
            t.fill_(float("nan"))
    m.step_grouped()
    torch.cuda.synchronize()
    for a, b in zip(ref, m.outputs()):
        assert torch.equal(a, b)
    g = m.capture()
    for i in range(3):
        for L in m.layers:
            for t in L.out.values():
                t.fill_(float("nan"))
        torch.cuda.synchronize()
        announce(f"decode {op} graph replay {i}")
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(ref, m.outputs()):
            assert torch.equal(a, b), i
    # first projection of layer 0 against the oracle
    W, s = m.layers[0].w["q"]
    y = m.layers[0].out["q"].cpu().numpy()
    x = m.x0.cpu().numpy()
    if op == "int4gemv":
        ex, S = orc.exact_w4(W.cpu().numpy(), s.cpu().numpy(), x)
    else:
        ex, S = orc.exact_w8(W.cpu().numpy(), s.cpu().numpy(), x)
    assert orc.arith_ratio(y, ex, S, x.size).max() <= 1.0
