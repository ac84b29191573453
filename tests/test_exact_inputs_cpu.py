"""CPU pins of the exact-input expectations (oracle.expect_exact_*), which
the GPU tests in test_gpu_exact.py compare every variant with bit for bit.

* The conditions are enforced: a scale that is not a power of two (or out
  of range), x outside {-1, 0, +1}, K past 131072, or W not a multiple of
  2^-6 raise.
* The expectation equals an independent computation in Python integers
  (units of 2^-6 for INT4 and FP16/FP32, of the row scale for INT8), cast
  once to the output type.
* Under the conditions every FP32 summation order gives the exact value:
  sequential, reversed, numpy's pairwise sum, and the kernels' order (16-
  or 32-element chunks, then a tree over lanes) all agree bit for bit.
* A planted mistake that the fixed accumulation bound cannot see at large
  K, one dropped 16-byte chunk of weights per row at K = 131072, changes
  the fp16 output of (nearly) every row: the exact-input check catches it.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc


def _w4_inputs(rng, N, K, exps=(-6, -5, -4, -3, -2)):
    wp = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    e = rng.choice(exps, size=(N, K // 128))
    scale = np.ldexp(1.0, e).astype(np.float16)
    x = rng.choice(np.array([-1.0, 0.0, 1.0], dtype=np.float16), size=K)
    return wp, scale, x


def _w8_inputs(rng, N, K):
    wq = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    scale = np.ldexp(1.0, rng.integers(-8, 1, size=N)).astype(np.float32)
    x = rng.choice(np.array([-1.0, 0.0, 1.0], dtype=np.float16), size=K)
    return wq, scale, x


def _gemv_inputs(rng, N, K, dtype):
    q = rng.integers(-8, 9, size=(N, K))
    e = rng.integers(2, 7, size=(N, K))
    W = np.ldexp(q.astype(np.float64), -e).astype(dtype)
    x = rng.choice(np.array([-1.0, 0.0, 1.0], dtype=dtype), size=K)
    return W, x


def test_conditions_are_enforced():
    rng = np.random.default_rng(0)
    wp, s, x = _w4_inputs(rng, 2, 256)
    with pytest.raises(ValueError, match="power of two"):
        orc.expect_exact_w4(wp, (s * np.float16(3)).astype(np.float16), x)
    with pytest.raises(ValueError, match="2\\^-6, 2\\^-2"):
        orc.expect_exact_w4(wp, np.full_like(s, 0.5), x)
    with pytest.raises(ValueError, match="x must lie"):
        orc.expect_exact_w4(wp, s, (x * np.float16(2)).astype(np.float16))
    with pytest.raises(ValueError, match="K = "):
        orc.expect_exact_w4(np.zeros((1, 131072), np.uint8),
                            np.full((1, 2048), 0.25, np.float16),
                            np.zeros(262144, np.float16))
    wq, s8, x8 = _w8_inputs(rng, 2, 64)
    with pytest.raises(ValueError, match="power of two"):
        orc.expect_exact_w8(wq, (s8 * 3).astype(np.float32), x8)
    with pytest.raises(ValueError, match="2\\^-8, 1"):
        orc.expect_exact_w8(wq, np.full_like(s8, 2.0), x8)
    W, xg = _gemv_inputs(rng, 2, 64, np.float16)
    with pytest.raises(ValueError, match="multiples of 2\\^-6"):
        orc.expect_exact_gemv((W + np.float16(2 ** -8)).astype(np.float16), xg)


def _int_w4(wp, scale, x):
    """Row sums in units of 2^-6 with Python integers."""
    q = orc.unpack_w(wp)          # exhaustively pinned against the closed form
    units = (scale.astype(np.float64) * 64).astype(np.int64)
    out = []
    for n in range(q.shape[0]):
        tot = 0
        for k in range(q.shape[1]):
            tot += int(q[n, k]) * int(units[n, k // 128]) * int(x[k])
        out.append(Fraction(tot, 64))
    return out


@pytest.mark.parametrize("N,K", [(3, 128), (5, 384), (2, 1024)])
def test_w4_expectation_is_the_exact_integer_sum(N, K):
    rng = np.random.default_rng(N * 1000 + K)
    wp, s, x = _w4_inputs(rng, N, K)
    want = np.array([float(v) for v in _int_w4(wp, s, x)]).astype(np.float16)
    got = orc.expect_exact_w4(wp, s, x)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("N,K", [(3, 16), (4, 100), (2, 999)])
def test_w8_expectation_is_the_exact_integer_sum(N, K):
    rng = np.random.default_rng(N * 1000 + K)
    wq, s, x = _w8_inputs(rng, N, K)
    tot = wq.astype(np.int64) @ x.astype(np.int64)
    want = np.array([float(Fraction(int(t)) * Fraction(float(sc)))
                     for t, sc in zip(tot, s)]).astype(np.float16)
    got = orc.expect_exact_w8(wq, s, x)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_gemv_expectation_is_the_exact_integer_sum(dtype):
    rng = np.random.default_rng(7)
    W, x = _gemv_inputs(rng, 4, 300, dtype)
    units = (W.astype(np.float64) * 64).astype(np.int64)
    tot = units @ x.astype(np.int64)
    want = np.array([float(Fraction(int(t), 64)) for t in tot]).astype(dtype)
    got = orc.expect_exact_gemv(W, x)
    assert got.dtype == dtype and np.array_equal(got, want)


def _fp32_orders(terms: np.ndarray) -> list[np.float32]:
    """The same float32 terms summed in several orders."""
    t = terms.astype(np.float32)
    seq = np.float32(0)
    for v in t:
        seq = np.float32(seq + v)
    rev = np.float32(0)
    for v in t[::-1]:
        rev = np.float32(rev + v)
    pairwise = np.sum(t, dtype=np.float32)
    # the kernels: each lane sums its chunks, then a tree over 64 lanes
    lanes = t.reshape(-1, 64, 32).sum(axis=2, dtype=np.float32).sum(axis=0, dtype=np.float32)
    while lanes.size > 1:
        lanes = (lanes[0::2] + lanes[1::2]).astype(np.float32)
    return [seq, rev, np.float32(pairwise), np.float32(lanes[0])]


def test_every_fp32_order_is_exact_under_the_conditions():
    rng = np.random.default_rng(11)
    K = 131072
    wp, s, x = _w4_inputs(rng, 1, K)
    q = orc.unpack_w(wp)[0].astype(np.float64)
    terms = q * np.repeat(s[0].astype(np.float64), 128) * x.astype(np.float64)
    exact = float(np.sum(terms))        # float64 sum of exact multiples of 2^-6: exact
    assert exact == float(sum(Fraction(v) for v in terms))
    sums = _fp32_orders(terms)
    assert all(float(v) == exact for v in sums), [float(v) for v in sums]
    assert np.float16(exact) == orc.expect_exact_w4(wp, s, x)[0]


@pytest.mark.parametrize("op", ["int4gemv", "qgemv"])
def test_one_dropped_chunk_at_k131072_fails_the_exact_check(op):
    """A kernel that skipped one 16-byte chunk of weights per row (32 INT4
    or 16 INT8 elements of 131072) passes the TOL_K bound but not the
    exact-input comparison."""
    rng = np.random.default_rng(5)
    N, K = 8, 131072
    if op == "int4gemv":
        wp, s, x = _w4_inputs(rng, N, K)
        want = orc.expect_exact_w4(wp, s, x)
        ex, S = orc.exact_w4(wp, s, x)
        bad = wp.copy()
        bad[:, 100 * 16:101 * 16] = 0             # chunk 100 of every row: q = 0
        wrong = orc.exact_w4(bad, s, x)[0].astype(np.float16)
    else:
        wq, s, x = _w8_inputs(rng, N, K)
        want = orc.expect_exact_w8(wq, s, x)
        ex, S = orc.exact_w8(wq, s, x)
        bad = wq.copy()
        bad[:, 100 * 16:101 * 16] = 0
        wrong = orc.exact_w8(bad, s, x)[0].astype(np.float16)
    # the bound does not see the missing chunk ...
    assert orc.arith_ratio(wrong, ex, S, K).max() <= 1.0
    # ... the exact comparison does, on nearly every row
    differ = int(np.count_nonzero(wrong.view(np.uint16) != want.view(np.uint16)))
    assert differ >= N - 1, differ


# ------------------------------------------- the timed CPU baseline ports
@pytest.mark.parametrize("threads", [1, 4])
@pytest.mark.parametrize("N,K", [(1, 128), (37, 4096), (256, 1024), (5, 16512)])
def test_cpu_port_w4_meets_the_bound_and_is_exact_on_exact_inputs(N, K, threads):
    """orc_int4_gemv_cpu (the C + OpenMP GEMV bench.py times as the CPU
    baseline) computes the same GEMV: within the bound on quantized N(0,1)
    data in every input mode, bit for bit on exact inputs, and the same
    bits for any thread count."""
    rng = np.random.default_rng(N + K)
    for mode_w, mode_x in ((0.02, 1.0), (1e-4, 1e-4), (10.0, 10.0)):
        W = (rng.standard_normal((N, K)) * mode_w).astype(np.float16)
        wp, s = orc.quantize_w4(W)
        x = (rng.standard_normal(K) * mode_x).astype(np.float16)
        y = orc.gemv_w4_cpu(wp, s, x, threads)
        ex, S = orc.exact_w4(wp, s, x)
        fits = np.abs(ex) <= 65504
        assert orc.arith_ratio(y[fits], ex[fits], S[fits], K).max(initial=0) <= 1.0
        assert np.array_equal(y.view(np.uint16), orc.gemv_w4_cpu(wp, s, x, 1).view(np.uint16))
    wp, s, x = _w4_inputs(rng, N, K)
    y = orc.gemv_w4_cpu(wp, s, x, threads)
    assert np.array_equal(y.view(np.uint16), orc.expect_exact_w4(wp, s, x).view(np.uint16))


@pytest.mark.parametrize("threads", [1, 4])
@pytest.mark.parametrize("N,K", [(1, 1), (16, 13), (37, 4096), (5, 16400)])
def test_cpu_port_w8_meets_the_bound_and_is_exact_on_exact_inputs(N, K, threads):
    rng = np.random.default_rng(N + K)
    for mode_w, mode_x in ((0.02, 1.0), (1e-4, 1e-4), (10.0, 10.0)):
        W = (rng.standard_normal((N, K)) * mode_w).astype(np.float16)
        wq, s = orc.quantize_w8(W)
        x = (rng.standard_normal(K) * mode_x).astype(np.float16)
        y = orc.gemv_w8_cpu(wq, s, x, threads)
        ex, S = orc.exact_w8(wq, s, x)
        fits = np.abs(ex) <= 65504
        assert orc.arith_ratio(y[fits], ex[fits], S[fits], K).max(initial=0) <= 1.0
        assert np.array_equal(y.view(np.uint16), orc.gemv_w8_cpu(wq, s, x, 1).view(np.uint16))
    wq, s, x = _w8_inputs(rng, N, K)
    y = orc.gemv_w8_cpu(wq, s, x, threads)
    assert np.array_equal(y.view(np.uint16), orc.expect_exact_w8(wq, s, x).view(np.uint16))


def test_cpu_port_rejects_a_planted_mistake():
    """The check above is not vacuous: the port's output with one weight
    byte changed fails the exact comparison."""
    rng = np.random.default_rng(9)
    wp, s, x = _w4_inputs(rng, 8, 4096)
    s[:, 0] = np.float16(0.25)             # group 0 of every row: the largest scale
    x[14] = np.float16(1.0)
    bad = wp.copy()
    bad[:, 7] ^= 0x01                      # element 14 of every row: q moves by 1
    y = orc.gemv_w4_cpu(bad, s, x, 2)
    want = orc.expect_exact_w4(wp, s, x)
    assert np.count_nonzero(y.view(np.uint16) != want.view(np.uint16)) == 8
