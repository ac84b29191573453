"""The eager fast path's acceptance rule (csrc/cq_pyfast.cpp), on CPU
tensors: a valid operand set is accepted and every single defect that the
checked path of ext.py rejects -- each operand's rank, size, dtype,
contiguity, layout and device -- is refused, for the three operators.  With
require_gpu (the rule the launch path applies) CPU tensors are never
accepted, so nothing here launches.  Also: the module's source stamp,
unknown variants and non-tensor operands are "not taken" (no exception),
and the checked path still raises its messages on CPU tensors."""
from __future__ import annotations

import pytest
import torch

from cudalab_amd import _capi
from cudalab_amd.build import build, source_hash


@pytest.fixture(scope="module")
def exts():
    return {op: build(op) for op in ("int4gemv", "qgemv", "gemv")}


def test_module_carries_the_tree_stamp():
    assert _capi.fast_module().src_hash == source_hash()


def _nc(t):
    """Same shape and dtype, not contiguous."""
    big = torch.zeros(*t.shape[:-1], 2 * t.shape[-1], dtype=t.dtype)
    return big[..., ::2]


def _meta(t):
    return torch.empty(t.shape, dtype=t.dtype, device="meta")


def _mutations(ops, base):
    """(description, operands) for every single-operand defect of `base`
    (a dict name -> tensor; `ops` the operand order of the call)."""
    out = []
    for name in ops:
        t = base[name]
        bad = {
            "rank+1": t.unsqueeze(0),
            "flat" if t.dim() == 2 else "rank2": t.reshape(-1) if t.dim() == 2 else t.view(1, -1),
            "not contiguous": _nc(t),
            "on another device": _meta(t),
            "sparse": t.to_sparse(),
        }
        for dt in (torch.uint8, torch.int8, torch.float16, torch.float32, torch.bfloat16):
            if dt != t.dtype:
                bad[f"dtype {dt}"] = torch.zeros(t.shape, dtype=dt)
        # one dimension larger and one smaller
        for d in range(t.dim()):
            for delta in (1, -1):
                shape = list(t.shape)
                shape[d] += delta
                if shape[d] >= 0:
                    bad[f"dim{d}{delta:+d}"] = torch.zeros(shape, dtype=t.dtype)
        for what, tb in bad.items():
            args = dict(base)
            args[name] = tb
            out.append((f"{name} {what}", [args[o] for o in ops]))
    return out


def _int4_base(N=8, K=256):
    return {"W": torch.zeros(N, K // 2, dtype=torch.uint8),
            "s": torch.zeros(N, K // 128, dtype=torch.float16),
            "x": torch.zeros(K, dtype=torch.float16),
            "out": torch.zeros(N, dtype=torch.float16)}


def _q8_base(N=8, K=48):
    return {"W": torch.zeros(N, K, dtype=torch.int8),
            "s": torch.zeros(N, dtype=torch.float32),
            "x": torch.zeros(K, dtype=torch.float16),
            "out": torch.zeros(N, dtype=torch.float16)}


def _gemv_base(dtype, N=8, K=40):
    return {"W": torch.zeros(N, K, dtype=dtype), "x": torch.zeros(K, dtype=dtype),
            "out": torch.zeros(N, dtype=dtype)}


@pytest.mark.parametrize("op", ["int4gemv", "qgemv"])
def test_quant_rule_accepts_valid_and_refuses_every_defect(exts, op):
    fast = exts[op]._fast
    base = _int4_base() if op == "int4gemv" else _q8_base()
    ops = ("W", "s", "x", "out")
    assert fast.accepts(*[base[o] for o in ops], False)
    assert not fast.accepts(*[base[o] for o in ops], True)      # CPU tensors
    muts = _mutations(ops, base)
    assert len(muts) > 40
    for what, args in muts:
        assert not fast.accepts(*args, False), f"{op}: accepted {what}"


def test_int4_rule_refuses_k_not_multiple_of_128(exts):
    fast = exts["int4gemv"]._fast
    W = torch.zeros(8, 32, dtype=torch.uint8)          # K = 64
    assert not fast.accepts(W, torch.zeros(8, 0, dtype=torch.float16),
                            torch.zeros(64, dtype=torch.float16),
                            torch.zeros(8, dtype=torch.float16), False)
    assert not fast.accepts(torch.zeros(0, 128, dtype=torch.uint8),
                            torch.zeros(0, 2, dtype=torch.float16),
                            torch.zeros(256, dtype=torch.float16),
                            torch.zeros(0, dtype=torch.float16), False)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["f16", "f32"])
def test_gemv_rule_accepts_valid_and_refuses_every_defect(exts, dtype):
    fast = exts["gemv"]._fast
    base = _gemv_base(dtype)
    ops = ("W", "x", "out")
    assert fast.gemv_accepts(*[base[o] for o in ops], False)
    assert not fast.gemv_accepts(*[base[o] for o in ops], True)
    for what, args in _mutations(ops, base):
        assert not fast.gemv_accepts(*args, False), f"gemv {dtype}: accepted {what}"
    # the quantized rule never accepts on the gemv launcher, and vice versa
    assert not fast.accepts(*[base[o] for o in ("W", "x", "x", "out")], False)
    assert not exts["int4gemv"]._fast.gemv_accepts(*[base[o] for o in ops], False)


def test_not_taken_on_cpu_tensors_unknown_variants_and_non_tensors(exts):
    b = _int4_base()
    fast = exts["int4gemv"]._fast
    args = (b["W"], b["s"], b["x"], b["out"])
    assert fast.into("int4gemv_cdna4", *args) is False
    assert fast.forward("int4gemv_cdna4", *args[:3]) is None
    assert fast.into("no_such_variant", *args) is False
    assert fast.into(17, *args) is False
    assert fast.into("int4gemv_cdna4", None, b["s"], b["x"], b["out"]) is False
    assert fast.into("int4gemv_cdna4", [1, 2], b["s"], b["x"], b["out"]) is False
    assert fast.forward("int4gemv_cdna4", b["W"], 3.0, b["x"]) is None
    g = _gemv_base(torch.float16)
    assert exts["gemv"]._fast.gemv_into("gemv_cdna4", g["W"], g["x"], g["out"]) is False
    assert exts["gemv"]._fast.gemv_forward("gemv_cdna4", g["W"], g["x"]) is None
    assert fast.cached() == 0


def test_checked_path_still_raises_after_the_fast_path_declines(exts):
    b = _int4_base()
    with pytest.raises(RuntimeError, match="CUDA 张量"):
        exts["int4gemv"].forward_into("int4gemv_cdna4", b["W"], b["s"], b["x"], b["out"])
    with pytest.raises(RuntimeError, match="未知 int4gemv 变体"):
        exts["int4gemv"].forward_into("nope", b["W"], b["s"], b["x"], b["out"])
    with pytest.raises(RuntimeError, match="必须是 2 维"):
        exts["int4gemv"].forward("int4gemv_cdna4", b["W"].view(-1), b["s"], b["x"])
    g = _gemv_base(torch.float32)
    with pytest.raises(RuntimeError, match="CUDA 张量"):
        exts["gemv"].forward("gemv_cdna4", g["W"], g["x"])


def test_knows_exactly_the_names_the_checked_path_accepts(exts):
    """The launcher's names are the checked path's: every registered
    variant (quarantined ones included) and every alias."""
    for op, e in exts.items():
        names = e.all_variants() + list(e.aliases())
        assert names
        for name in names:
            e._lookup(name)
            assert e._fast.knows(name), (op, name)
        for other in ("", "int4gemv", "gemv_cdna4 ", "qgemv_cdna4x"):
            assert not e._fast.knows(other), (op, other)
        assert not e._fast.knows(None)


def test_grouped_not_taken_without_launching(exts):
    """The grouped fast path takes only lists or tuples of 4-item problems
    of GPU tensors; anything else is "not taken" -- and an iterator is left
    unconsumed for the checked path."""
    b = _int4_base()
    prob = (b["W"], b["s"], b["x"], b["out"])
    fast = exts["int4gemv"]._fast
    assert fast.grouped("int4gemv_cdna4", [prob, prob]) is False     # CPU tensors
    assert fast.grouped("int4gemv_cdna4", []) is False
    assert fast.grouped("int4gemv_cdna4", [prob[:3]]) is False
    assert fast.grouped("int4gemv_cdna4", [list(prob) + [None]]) is False
    assert fast.grouped("int4gemv_cdna4", [(None,) * 4]) is False
    assert fast.grouped("int4gemv_cdna4", prob[0]) is False
    assert fast.grouped("no_such_variant", [prob]) is False
    it = iter([prob])
    assert fast.grouped("int4gemv_cdna4", it) is False
    assert next(it) is prob                                        # not consumed
    assert exts["gemv"]._fast.grouped("gemv_cdna4", [prob]) is False
    with pytest.raises(RuntimeError, match="CUDA 张量"):
        exts["int4gemv"].forward_grouped("int4gemv_cdna4", iter([prob]))


def test_module_carries_the_torch_abi_stamp():
    from cudalab_amd.build import fast_abi_stamp
    assert _capi.fast_module().abi_stamp == fast_abi_stamp()
    assert f"torch={torch.__version__};" in fast_abi_stamp()


def test_module_built_against_another_torch_is_refused(monkeypatch):
    """A module whose ABI stamp differs from this process's torch is refused
    on load, like a module built from other sources."""
    monkeypatch.setattr(_capi, "_fast", None)
    monkeypatch.setattr(_capi, "fast_abi_stamp",
                        lambda: "torch=0.0.0;cxx11abi=0;flags=0")
    with pytest.raises(_capi.StaleLibrary, match="another torch"):
        _capi.fast_module()


def test_operators_work_without_the_fast_module(monkeypatch):
    """With the fast-path module unusable, an operator warns once and takes
    the checked path for every call: the launcher declines everything and
    the checked path still raises the reference's messages."""
    from cudalab_amd import ext as ext_mod

    def missing():
        raise _capi.LibraryMissing("no _cqfast here")

    monkeypatch.setattr(_capi, "fast_module", missing)
    monkeypatch.setattr(ext_mod, "_fast_warned", False)
    with pytest.warns(RuntimeWarning, match="checked path"):
        e = ext_mod.Int4gemvExt()
    assert isinstance(e._fast, ext_mod._DeclineAll)
    W = torch.zeros(8, 128, dtype=torch.uint8)
    s = torch.zeros(8, 2, dtype=torch.float16)
    x = torch.zeros(256, dtype=torch.float16)
    out = torch.zeros(8, dtype=torch.float16)
    assert e._fast.into("int4gemv_cdna4", W, s, x, out) is False
    assert e._fast.forward("int4gemv_cdna4", W, s, x) is None
    assert e._fast.grouped("int4gemv_cdna4", [(W, s, x, out)]) is False
    with pytest.raises(RuntimeError, match="CUDA 张量"):
        e.forward_into("int4gemv_cdna4", W, s, x, out)
    g = ext_mod.GemvExt()          # second operator: no second warning
    assert isinstance(g._fast, ext_mod._DeclineAll)
