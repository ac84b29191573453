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


def test_decode_grouped_query_kv(cuda):
    """A 70B-shaped layer pair (H = 8192, I = 28672, k/v width 1024): k and v
    are narrower than q, o reads v repeated per query head group, and the
    down projection (K = 28672) runs the K-tiled kernel.  Sequential,
    grouped and graph-replayed steps agree bit for bit, and o's input is
    the repeated v."""
    from cudalab_amd.decode import HEAD_DIM, MODELS, DecodeModel
    cfg = MODELS["70b"]
    announce("decode int4gemv 70b-shaped, 2 layers")
    m = DecodeModel("int4gemv", layers=2, seed=5, hidden=cfg["hidden"],
                    inter=cfg["inter"], kv=cfg["kv"])
    assert m.ext.describe(m.variant, m.layers[0].w["down"][0],
                          m.layers[0].out["up"])["kernel"] == "tiled"
    m.step_sequential()
    torch.cuda.synchronize()
    ref = m.outputs()
    assert all(torch.isfinite(t).all() for t in ref)
    L = m.layers[0]
    rep = cfg["hidden"] // cfg["kv"]
    v = L.out["v"].view(-1, HEAD_DIM)
    assert torch.equal(L.out["o_in"].view(-1, rep, HEAD_DIM),
                       v[:, None, :].expand(-1, rep, HEAD_DIM))
    m.step_grouped()
    torch.cuda.synchronize()
    for a, b in zip(ref, m.outputs()):
        assert torch.equal(a, b)
    g = m.capture()
    for i in range(2):
        for Ly in m.layers:
            for t in Ly.out.values():
                t.fill_(float("nan"))
        torch.cuda.synchronize()
        announce(f"decode 70b-shaped graph replay {i}")
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(ref, m.outputs()):
            assert torch.equal(a, b), i
    # the tiled down projection of layer 0 against the oracle
    W, s = L.w["down"]
    x = L.out["up"].cpu().numpy()
    ex, S = orc.exact_w4(W.cpu().numpy(), s.cpu().numpy(), x)
    assert orc.arith_ratio(L.out["down"].cpu().numpy(), ex, S, x.size).max() <= 1.0


def test_decode_rejects_bad_kv(cuda):
    from cudalab_amd.decode import DecodeModel
    with pytest.raises(ValueError, match="k/v width"):
        DecodeModel("int4gemv", layers=1, hidden=4096, inter=4096, kv=1000)
