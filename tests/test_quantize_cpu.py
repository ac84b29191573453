"""CPU checks of the on-device quantizers' arithmetic and of their C entry
points (no kernel is launched).

The scale has two forms, as the reference's `amax / qmax` (a tensor
divided by a Python number) is rounded by torch: one correctly rounded
division on the CPU, amax * fl(1/qmax) on a GPU.  Both are checked.

The HIP kernels estimate q = rint(fl(w / s)) as the round-half-even
integer k of the exact product w * r (one fma), r = v_rcp_f32(s), and
recompute with the correctly rounded division only for 8-element chunks
where w * r - k (one more fma) is within 2^-18 (INT4) or 2^-13 (INT8) of
+-1/2; they pack through 32-bit sums of the float bit patterns.
`_emulate_q` and the `_pack_*` helpers restate that arithmetic in numpy
with r moved up to two float32 steps from the correctly rounded 1/s
(v_rcp_f32 is specified to 1 ulp), and the tests check it against the
oracle's quantizers (the reference's formula,
cudalab/int4gemv_quantize.py:61-114, cudalab/qgemv_quantize.py:33-64) on
random and crafted inputs, ties included.  Dropping the recompute (a
planted mistake) must fail."""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from cudalab_amd import _capi
from oracle import oracle as orc

import quant_cases as qc

MAGIC_BITS = np.uint32(0x4B400000)          # bits of 1.5 * 2^23
PACK4_ADD = np.uint32(((136 - 17 * 0x4B400000) * 0x01010101) % 2 ** 32)
PACK8_ADD = np.uint32(((128 - 0x4B400000) * 0x01010101) % 2 ** 32)
NEAR = {7: np.float32(0.5 - 2.0 ** -18), 127: np.float32(0.5 - 2.0 ** -13)}


def _step(r: np.ndarray, n: int) -> np.ndarray:
    out = r.copy()
    d = np.float32(np.inf if n > 0 else -np.inf)
    for _ in range(abs(n)):
        out = np.nextafter(out, d).astype(np.float32)
    return out


def _emulate_q(W16: np.ndarray, qmax: int, group: int, rcp_steps: int,
               recompute: bool = True, rcp_scale: bool = False):
    """The kernels' arithmetic: returns (q int64 (N, K), s float32 per
    group, number of 8-element chunks that took the recompute).

    m = fma(w, r, 1.5 * 2^23) rounds the exact product w * r once: in
    float64 the product of an fp16 and an fp32 is exact, and rint of it is
    the round-half-even integer k.  d = fma(w, r, -k) is w * r - k (exact in
    float64) rounded once to float32."""
    N, K = W16.shape
    w = W16.astype(np.float32).reshape(N, K // group, group)
    amax = np.abs(w).max(axis=2)
    if rcp_scale:
        s = (amax * (np.float32(1) / np.float32(qmax))).astype(np.float32)
    else:
        s = (amax / np.float32(qmax)).astype(np.float32)
    with np.errstate(divide="ignore"):
        r = np.where(s == 0, np.float32(0), np.float32(1) / s).astype(np.float32)
    r = np.where(s == 0, np.float32(0), _step(r, rcp_steps)).astype(np.float32)
    p = w.astype(np.float64) * r.astype(np.float64)[:, :, None]
    k = np.rint(p)
    d = (p - k).astype(np.float32)
    q = k.astype(np.int64)
    near = (np.abs(d) > NEAR[qmax]).reshape(N, K // 8, 8).any(axis=2)
    if recompute:
        with np.errstate(divide="ignore", invalid="ignore"):
            exact = np.rint((w / np.where(s == 0, np.float32(1), s)[:, :, None])
                            .astype(np.float32))
        exact = np.clip(exact, -qmax, qmax)
        exact[np.broadcast_to((s == 0)[:, :, None], exact.shape)] = 0
        qc8 = q.reshape(N, K // 8, 8)
        ex8 = exact.reshape(N, K // 8, 8).astype(np.int64)
        qc8[near] = ex8[near]
        q = qc8.reshape(N, K // group, group)
    return q.reshape(N, K), s, int(near.sum())


def _bits(q: np.ndarray) -> np.ndarray:
    """bits(m) = bits(1.5 * 2^23) + q, as the kernels hold it."""
    return (MAGIC_BITS.astype(np.int64) + q).astype(np.uint32)


def _pack_nibbles(q: np.ndarray) -> np.ndarray:
    """The kernels' INT4 packing: (N, K) ints in [-7, 7] -> uint8 (N, K/2),
    through 32-bit sums of the magic bit patterns."""
    N, K = q.shape
    b = _bits(q).reshape(N, K // 8, 8)
    acc = np.full((N, K // 8), PACK4_ADD, dtype=np.uint32)
    for j in range(4):
        pj = (b[:, :, 2 * j] + (b[:, :, 2 * j + 1] << np.uint32(4))).astype(np.uint32)
        acc = (acc + (pj << np.uint32(8 * j))).astype(np.uint32)
    acc ^= np.uint32(0x88888888)
    return acc.view(np.uint8).reshape(N, K // 2)


def _pack_bytes(q: np.ndarray) -> np.ndarray:
    """The kernels' INT8 packing: (N, K) ints in [-127, 127], K % 4 == 0 ->
    int8 (N, K)."""
    N, K = q.shape
    b = _bits(q).reshape(N, K // 4, 4)
    acc = (b[:, :, 0] + (b[:, :, 1] << np.uint32(8)) + (b[:, :, 2] << np.uint32(16))
           + (b[:, :, 3] << np.uint32(24)) + PACK8_ADD).astype(np.uint32)
    acc ^= np.uint32(0x80808080)
    return acc.view(np.int8).reshape(N, K)


def _emulate_w4(W16, rcp_steps, recompute=True, rcp_scale=False):
    q, s, n_near = _emulate_q(W16, 7, 128, rcp_steps, recompute, rcp_scale)
    return _pack_nibbles(np.clip(q, -8, 7)), s.astype(np.float16), n_near


def _emulate_w8(W16, rcp_steps, recompute=True, rcp_scale=False):
    N, K = W16.shape
    q, s, n_near = _emulate_q(W16, 127, K, rcp_steps, recompute, rcp_scale)
    return _pack_bytes(q), s.reshape(N), n_near


def test_packing_identities_exhaustive():
    """The bit-pattern packing equals the nibble/byte contract for every
    value pair (INT4) and value (INT8) the quantizers produce."""
    ks = np.arange(-7, 8)
    lo, hi = np.meshgrid(ks, ks, indexing="ij")
    q = np.stack([lo.ravel(), hi.ravel()], axis=1).reshape(1, -1)
    q = np.concatenate([q, np.zeros((1, (-q.shape[1]) % 8), dtype=q.dtype)], axis=1)
    assert np.array_equal(_pack_nibbles(q), orc.pack_q(q))
    q8 = np.arange(-127, 129).reshape(1, -1)
    q8[0, -1] = 0
    assert np.array_equal(_pack_bytes(q8), q8.astype(np.int8))


@pytest.mark.parametrize("rcp_scale", [False, True], ids=["div", "rcp"])
@pytest.mark.parametrize("steps", [-2, -1, 0, 1, 2])
@pytest.mark.parametrize("case", sorted(qc.all_cases(7)))
def test_int4_estimate_with_recompute_is_exact(case, steps, rcp_scale):
    W = qc.all_cases(7)[case]
    wp, s16 = orc.quantize_w4(W, rcp=rcp_scale)
    ewp, es16, _ = _emulate_w4(W, steps, rcp_scale=rcp_scale)
    assert np.array_equal(ewp, wp), case
    assert np.array_equal(es16.view(np.uint16), s16.view(np.uint16)), case


@pytest.mark.parametrize("rcp_scale", [False, True], ids=["div", "rcp"])
@pytest.mark.parametrize("steps", [-2, -1, 0, 1, 2])
@pytest.mark.parametrize("case", sorted(qc.all_cases(127)))
def test_int8_estimate_with_recompute_is_exact(case, steps, rcp_scale):
    W = qc.all_cases(127)[case]
    wq, s = orc.quantize_w8(W, rcp=rcp_scale)
    ewq, es, _ = _emulate_w8(W, steps, rcp_scale=rcp_scale)
    assert np.array_equal(ewq, wq), case
    assert np.array_equal(es.view(np.uint32), s.view(np.uint32)), case


@pytest.mark.parametrize("steps", [-2, 0, 2])
def test_estimate_exact_on_many_random_groups(steps):
    """2^21 random elements per quantizer, several magnitudes, both scale
    forms."""
    for std in (1.0, 0.02, 1e-4, 300.0):
        W = qc.random_rows(1024, 2048, seed=int(std * 1000) + 7, std=std)
        for rcp in (False, True):
            wp, _ = orc.quantize_w4(W, rcp=rcp)
            assert np.array_equal(_emulate_w4(W, steps, rcp_scale=rcp)[0], wp), std
            wq, _ = orc.quantize_w8(W, rcp=rcp)
            assert np.array_equal(_emulate_w8(W, steps, rcp_scale=rcp)[0], wq), std


def _nearest_f32(fr: Fraction) -> np.float32:
    """The float32 nearest to a positive rational (ties to even), by exact
    comparison with the two float32 neighbours of its float64 rounding."""
    c = np.float32(float(fr))
    best = None
    for v in (np.nextafter(c, np.float32(0)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(v)) - fr)
        key = (d, int(np.array(v).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, v)
    return np.float32(best[1])


def test_scale_forms_pinned_over_every_fp16_amax():
    """Both scale forms against exact rational arithmetic, for every finite
    positive fp16 amax: the division form is the rational amax/qmax rounded
    once; the reciprocal form is fl(amax * fl(1/qmax)) with fl(1/qmax) the
    rounded rational 1/qmax (fl32(1/7) = 0x3E124925).  The forms differ for
    about half of the amax values with 7, so the choice matters."""
    h = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16)
    amax = h.astype(np.float32)
    for qmax in (7, 127):
        inv = _nearest_f32(Fraction(1, qmax))
        if qmax == 7:
            assert int(np.array(inv).view(np.uint32)) == 0x3E124925
        div = orc._scale(amax, qmax, rcp=False)
        rcp = orc._scale(amax, qmax, rcp=True)
        # float64 products of an 11-bit and a 24-bit significand are exact
        want_rcp = (amax.astype(np.float64) * np.float64(inv)).astype(np.float32)
        assert np.array_equal(rcp.view(np.uint32), want_rcp.view(np.uint32)), qmax
        for i in range(0, h.size, 97):            # exact rational spot checks
            assert div[i] == _nearest_f32(Fraction(float(amax[i])) / qmax)
            assert rcp[i] == _nearest_f32(Fraction(float(amax[i])) * Fraction(float(inv)))
        frac = float((div != rcp).mean())
        assert (0.4 < frac < 0.7) if qmax == 7 else (0.01 < frac < 0.2), (qmax, frac)


def test_torch_cpu_scale_is_the_division_form():
    """The reference's expression evaluated by torch on the CPU is the
    division form (and the forced forms of this build's torch path match
    the oracle's)."""
    import torch
    from cudalab_amd import int4gemv_quantize as q4, qgemv_quantize as q8
    W = torch.from_numpy(qc.random_rows(256, 1024, seed=21))
    for rcp in (None, False, True):
        a = q4.quantize_w_torch(W, rcp=rcp)
        b = orc.quantize_w4(W.numpy(), rcp=bool(rcp))
        assert np.array_equal(a[0].numpy(), b[0]) and np.array_equal(
            a[1].numpy().view(np.uint16), b[1].view(np.uint16)), rcp
        a = q8.quantize_w_torch(W, rcp=rcp)
        b = orc.quantize_w8(W.numpy(), rcp=bool(rcp))
        assert np.array_equal(a[0].numpy(), b[0]) and np.array_equal(
            a[1].numpy().view(np.uint32), b[1].view(np.uint32)), rcp
    for sem, rcp in (("cpu", False), ("gpu", True)):
        assert np.array_equal(q4.quantize_w(W, semantics=sem)[0].numpy(),
                              orc.quantize_w4(W.numpy(), rcp=rcp)[0]), sem
    with pytest.raises(ValueError, match="semantics"):
        q4.quantize_w(W, semantics="tpu")


def test_recompute_is_needed_and_rare():
    """Without the recompute the estimate is wrong on exact ties (the
    planted mistake fails).  On N(0, 1) fp16 weights about 0.3% of the
    8-element chunks take the recompute, most of them exact ties (an amax
    whose mantissa is a multiple of 7 makes s a short binary fraction)."""
    T4 = qc.ties(7, 96, seed=11)
    bad4, _, _ = _emulate_w4(T4, 1, recompute=False)
    assert not np.array_equal(bad4, orc.quantize_w4(T4)[0])
    T8 = qc.ties(127, 96, seed=11)
    bad8, _, _ = _emulate_w8(T8, 1, recompute=False)
    assert not np.array_equal(bad8, orc.quantize_w8(T8)[0])
    R = qc.random_rows(512, 4096, seed=3)
    _, _, n4 = _emulate_w4(R, 0)
    _, _, n8 = _emulate_w8(R, 0)
    chunks = R.size // 8
    assert n4 / chunks < 1e-2 and n8 / chunks < 1e-2, (n4, n8, chunks)


@pytest.mark.parametrize("rcp", [False, True], ids=["div", "rcp"])
def test_oracle_c_and_numpy_agree_on_crafted_cases(rcp):
    for case, W in qc.all_cases(7).items():
        a, b = orc.quantize_w4(W, rcp=rcp), orc.quantize_w4_c(W, rcp=rcp)
        assert np.array_equal(a[0], b[0]) and np.array_equal(
            a[1].view(np.uint16), b[1].view(np.uint16)), case
    for case, W in qc.all_cases(127).items():
        a, b = orc.quantize_w8(W, rcp=rcp), orc.quantize_w8_c(W, rcp=rcp)
        assert np.array_equal(a[0], b[0]) and np.array_equal(
            a[1].view(np.uint32), b[1].view(np.uint32)), case


def test_ties_round_to_even():
    """Closed form: with amax = 7 (s = 1 exactly) w = j + 1/2 quantizes to
    the even one of j, j + 1."""
    W = np.zeros((1, 128), dtype=np.float16)
    W[0, 0] = 7
    vals = np.arange(-7, 7) + 0.5
    W[0, 1:1 + vals.size] = vals
    q = orc.unpack_w(orc.quantize_w4(W)[0])[0, 1:1 + vals.size]
    want = np.where(np.floor(vals) % 2 == 0, np.floor(vals), np.floor(vals) + 1)
    assert np.array_equal(q, want.astype(np.int32))


# ----------------------------------------------------- C entry points, no GPU
def test_quantize_argument_errors_without_launch():
    lib = _capi.load()
    P, Q = 0x1000, 0x2000
    E = _capi.CQ_ERR_INVALID_ARG
    R = _capi.CQ_SCALE_RCP
    assert lib.cq_int4_quantize(None, P, Q, 4, 128, R, None) == E
    assert "null" in _capi.last_error()
    assert lib.cq_int4_quantize(P, None, Q, 4, 128, R, None) == E
    assert lib.cq_int4_quantize(P, P, None, 4, 128, R, None) == E
    assert lib.cq_int4_quantize(P, P, Q, 0, 128, R, None) == E
    assert lib.cq_int4_quantize(P, P, Q, 4, 0, R, None) == E
    assert lib.cq_int4_quantize(P, P, Q, 4, 200, R, None) == E
    assert "128" in _capi.last_error()
    assert lib.cq_int4_quantize(P + 1, P, Q, 4, 128, R, None) == E
    assert lib.cq_int4_quantize(P, P, Q + 1, 4, 128, R, None) == E
    assert lib.cq_int4_quantize(P, P, Q, 1 << 31, 128, R, None) == E
    assert lib.cq_int4_quantize(P, P, Q, 4, 128, 2, None) == E
    assert "scale_mode" in _capi.last_error()
    assert lib.cq_q8_quantize(None, P, Q, 4, 7, R, None) == E
    assert lib.cq_q8_quantize(P, P, Q, 4, 0, R, None) == E
    assert lib.cq_q8_quantize(P, P, Q + 2, 4, 7, R, None) == E   # fp32 scale
    assert lib.cq_q8_quantize(P + 1, P, Q, 4, 7, R, None) == E
    assert lib.cq_q8_quantize(P, P, Q, 4, 7, -1, None) == E


def test_quantize_overlapping_buffers_rejected_without_launch():
    """The kernels read w while other workgroups write the packed weights
    and the scales: in-place or overlapping buffers are argument errors
    (w is n*k*2 bytes; INT4 packed n*k/2 and scale n*(k/128)*2; INT8
    packed n*k and scale n*4)."""
    lib = _capi.load()
    E = _capi.CQ_ERR_INVALID_ARG
    R = _capi.CQ_SCALE_RCP
    W, Q, S = 0x100000, 0x200000, 0x300000                # n = 4, k = 128: w 1024 B
    for w, q, s in ((W, W, S), (W, W + 1020, S), (W, Q, W + 512), (W, Q, Q + 252)):
        assert lib.cq_int4_quantize(w, q, s, 4, 128, R, None) == E, (hex(w), hex(q), hex(s))
        assert "must not overlap" in _capi.last_error()
    for w, q, s in ((W, W + 1016, S), (W, Q, Q + 504)):   # INT8: packed 512 B
        assert lib.cq_q8_quantize(w, q, s, 4, 128, R, None) == E, (hex(q), hex(s))
        assert "must not overlap" in _capi.last_error()


@pytest.mark.parametrize("op,w,out,n,k,fast", [
    ("int4gemv", 0x1000, 0x2000, 4, 128, True),
    ("int4gemv", 0x1002, 0x2000, 4, 128, False),   # w not 16-byte aligned
    ("int4gemv", 0x1000, 0x2001, 4, 128, False),   # packed output not 4-byte
    ("int4gemv", 0x1000, 0x2004, 4, 256, True),
    ("qgemv", 0x1000, 0x2000, 4, 4096, True),
    ("qgemv", 0x1000, 0x2000, 4, 4100, False),     # k % 8
    ("qgemv", 0x1000, 0x2004, 4, 4096, False),     # output not 8-byte
    ("qgemv", 0x1008, 0x2000, 4, 4096, False),
])
def test_quantize_path_selection(op, w, out, n, k, fast):
    lib = _capi.load()
    assert lib.cq_quantize_vectorized(_capi.OPS[op], w, out, n, k) == int(fast)


def test_quantize_path_selection_rejects_other_ops():
    lib = _capi.load()
    assert lib.cq_quantize_vectorized(_capi.CQ_OP_GEMV_F16, 0x1000, 0x1000, 1, 8) == -1
