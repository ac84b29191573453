"""Pins of the CPU oracle (oracle/): each oracle function is checked against
something the mathematics fixes -- closed forms, exhaustive enumeration,
exact rational arithmetic, or IEEE conversions of numpy -- and the parity
gate is shown to reject planted mistakes (planted in CPU code here, never on
the GPU)."""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc


# ------------------------------------------------------------ nibbles

def _closed_form(b: int) -> tuple[int, int]:
    lo = b & 0xF
    hi = (b >> 4) & 0xF
    return (lo - 16 if lo >= 8 else lo), (hi - 16 if hi >= 8 else hi)


def test_unpack_all_256_bytes_numpy_and_c():
    wp = np.arange(256, dtype=np.uint8).reshape(1, 256)
    for q in (orc.unpack_w(wp), orc.unpack_w_c(wp)):
        assert q.shape == (1, 512)
        for b in range(256):
            assert (q[0, 2 * b], q[0, 2 * b + 1]) == _closed_form(b), b


def test_pack_is_inverse_of_unpack():
    wp = np.arange(256, dtype=np.uint8).reshape(2, 128)
    assert np.array_equal(orc.pack_q(orc.unpack_w(wp)), wp)
    vals = np.arange(-8, 8)
    lo = np.zeros((1, 32), np.int64)
    lo[0, 0::2] = vals
    hi = np.zeros((1, 32), np.int64)
    hi[0, 1::2] = vals
    assert np.array_equal(orc.unpack_w(orc.pack_q(lo))[0, 0::2], vals)
    assert np.array_equal(orc.unpack_w(orc.pack_q(hi))[0, 1::2], vals)
    with pytest.raises(ValueError):
        orc.pack_q(np.array([[8, 0]]))
    with pytest.raises(ValueError):
        orc.pack_q(np.array([[-9, 0]]))
    with pytest.raises(ValueError):
        orc.pack_q(np.zeros((1, 3), np.int64))


# ---------------------------------------------------- fp16 conversions

def test_h2d_all_65536_patterns():
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float64)
    got = np.array([L.orc_h2d(int(b)) for b in bits])
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


def test_f2h_matches_ieee_round_to_nearest_even():
    L = orc.lib()
    rng = np.random.default_rng(7)
    pats = rng.integers(0, 2 ** 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the fp16 range and on exact ties
    near = rng.integers(0x33000000, 0x47800000, size=200_000,
                        dtype=np.uint64).astype(np.uint32)
    ties = (near & ~np.uint32(0x1FFF)) | np.uint32(0x1000)
    edges = np.array([0, 0x80000000, 0x33000000, 0x33000001, 0x337fffff,
                      0x38800000, 0x387fffff, 0x477fe000, 0x477fefff,
                      0x477ff000, 0x477ff001, 0x7f800000, 0xff800000,
                      0x7fc00000, 0x3f800000], dtype=np.uint32)
    allp = np.concatenate([pats, near, ties, edges])
    f = allp.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f2h(float(v)) for v in f], dtype=np.uint16)
    isnan = np.isnan(f)
    assert np.array_equal(got[~isnan], want[~isnan])
    assert np.all((got[isnan] & 0x7C00) == 0x7C00) and np.all(got[isnan] & 0x3FF)


# ------------------------------------------------------- exact sums

def _frac_exact_w4(wp, scale, x):
    q = orc.unpack_w(wp)
    N, K = q.shape
    ex, S = [], []
    for n in range(N):
        tot = Fraction(0)
        ab = Fraction(0)
        for k in range(K):
            t = (q[n, k] * Fraction(float(scale[n, k // 128]))
                 * Fraction(float(x[k])))
            tot += t
            ab += abs(t)
        ex.append(float(tot))
        S.append(float(ab))
    return np.array(ex), np.array(S)


def _rand_case_w4(rng, N, K, x_scale=1.0, s_scale=0.01):
    wp = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    scale = (np.abs(rng.standard_normal((N, K // 128))) * s_scale).astype(np.float16)
    x = (rng.standard_normal(K) * x_scale).astype(np.float16)
    return wp, scale, x


@pytest.mark.parametrize("N,K,xs,ss", [(3, 128, 1.0, 0.01), (2, 256, 1e-4, 1e-4),
                                       (2, 384, 30.0, 2.0), (1, 128, 1e-6, 1e-3)])
def test_exact_w4_matches_fractions(N, K, xs, ss):
    rng = np.random.default_rng(N * 1000 + K)
    wp, scale, x = _rand_case_w4(rng, N, K, xs, ss)
    ex, S = orc.exact_w4(wp, scale, x)
    fex, fS = _frac_exact_w4(wp, scale, x)
    assert np.array_equal(ex, fex)
    assert np.array_equal(S, fS)


def test_exact_w4_closed_forms():
    # all nibbles +1 (byte 0x11), scale 1, x = 1 -> exact = K
    K = 4096
    wp = np.full((2, K // 2), 0x11, np.uint8)
    scale = np.ones((2, K // 128), np.float16)
    x = np.ones(K, np.float16)
    ex, S = orc.exact_w4(wp, scale, x)
    assert np.all(ex == K) and np.all(S == K)
    # one-hot x picks one dequantized weight: q[n,k] * s[n,k/128]
    rng = np.random.default_rng(3)
    wp, scale, _ = _rand_case_w4(rng, 4, 512)
    q = orc.unpack_w(wp)
    for k in (0, 1, 127, 128, 255, 511):
        x = np.zeros(512, np.float16)
        x[k] = 1
        ex, _ = orc.exact_w4(wp, scale, x)
        want = q[:, k] * scale[:, k // 128].astype(np.float64)
        assert np.array_equal(ex, want), k
    # -8 (byte 0x88) is representable in the packed format
    wp = np.full((1, 64), 0x88, np.uint8)
    ex, _ = orc.exact_w4(wp, np.ones((1, 1), np.float16), np.ones(128, np.float16))
    assert ex[0] == -8 * 128


def _frac_exact_w8(wq, scale, x):
    N, K = wq.shape
    ex, S = [], []
    for n in range(N):
        s = Fraction(float(scale[n]))
        tot = sum((int(wq[n, k]) * Fraction(float(x[k])) for k in range(K)),
                  Fraction(0)) * s
        ab = sum((abs(int(wq[n, k])) * abs(Fraction(float(x[k])))
                  for k in range(K)), Fraction(0)) * abs(s)
        ex.append(float(tot))
        S.append(float(ab))
    return np.array(ex), np.array(S)


@pytest.mark.parametrize("N,K", [(3, 13), (2, 64), (1, 1), (4, 300)])
def test_exact_w8_matches_fractions(N, K):
    rng = np.random.default_rng(N * 77 + K)
    wq = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    scale = (np.abs(rng.standard_normal(N)) * 0.003).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float16)
    ex, S = orc.exact_w8(wq, scale, x)
    fex, fS = _frac_exact_w8(wq, scale, x)
    assert np.array_equal(ex, fex)
    assert np.array_equal(S, fS)


def test_nonfinite_inputs_flag_nan():
    wp = np.zeros((1, 64), np.uint8)
    x = np.ones(128, np.float16)
    x[3] = np.inf
    ex, S = orc.exact_w4(wp, np.ones((1, 1), np.float16), x)
    assert np.isnan(ex[0]) and np.isnan(S[0])


# ------------------------------------------------ FP32 sequential ref

def test_ref_f32_w4_is_sequential_fp32():
    rng = np.random.default_rng(11)
    wp, scale, x = _rand_case_w4(rng, 3, 256)
    y32, y16 = orc.ref_f32_w4(wp, scale, x)
    q = orc.unpack_w(wp)
    for n in range(3):
        acc = np.float32(0)
        for k in range(256):
            w = np.float32(q[n, k]) * np.float32(scale[n, k // 128])
            acc = np.float32(acc + np.float32(w * np.float32(x[k])))
        assert acc == y32[n]
        assert np.float16(acc) == y16[n]


def test_ref_f32_w8_is_sequential_fp32():
    rng = np.random.default_rng(12)
    wq = rng.integers(-127, 128, size=(2, 45), dtype=np.int8)
    scale = np.array([0.0123, 3.5e-5], np.float32)
    x = rng.standard_normal(45).astype(np.float16)
    y32, _ = orc.ref_f32_w8(wq, scale, x)
    for n in range(2):
        acc = np.float32(0)
        for k in range(45):
            acc = np.float32(acc + np.float32(np.float32(wq[n, k]) * scale[n])
                             * np.float32(x[k]))
        assert acc == y32[n]


# -------------------------------------------------------- quantizers

def _w_modes(rng, N, K):
    yield "normal", (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    yield "unit", rng.standard_normal((N, K)).astype(np.float16)
    yield "tiny", (rng.standard_normal((N, K)) * 1e-4).astype(np.float16)
    yield "large", (rng.standard_normal((N, K)) * 10).astype(np.float16)
    z = (rng.standard_normal((N, K)) * 0.5).astype(np.float16)
    z[:, :128] = 0
    yield "zero_group", z


def test_quantize_w4_numpy_equals_c_and_closed_form():
    rng = np.random.default_rng(5)
    for name, W in _w_modes(rng, 6, 512):
        wp_n, s_n = orc.quantize_w4(W)
        wp_c, s_c = orc.quantize_w4_c(W)
        assert np.array_equal(wp_n, wp_c), name
        assert np.array_equal(s_n.view(np.uint16), s_c.view(np.uint16)), name
        g = W.astype(np.float32).reshape(6, 4, 128)
        s32 = (np.abs(g).max(axis=2) / np.float32(7)).astype(np.float32)
        assert np.array_equal(s_n, s32.astype(np.float16)), name
        q = orc.unpack_w(wp_n).reshape(6, 4, 128)
        assert np.abs(q).max() <= 7
        nz = s32 > 0
        err = np.abs(g - q * s32[:, :, None])
        assert np.all(err[nz] <= 0.5 * s32[nz][:, None] * (1 + 2.0 ** -20)), name
        assert np.all(q[~nz] == 0)


def test_quantize_w4_ties_round_half_to_even():
    # amax = 7 -> s32 = 1 exactly; W/s = k + 0.5 are exact ties
    W = np.zeros((1, 128), np.float16)
    W[0, :8] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]
    wp, s = orc.quantize_w4(W)
    assert s[0, 0] == 1.0
    q = orc.unpack_w(wp)[0, :8]
    assert list(q) == [7, 0, 2, 2, 0, -2, -2, 4]
    wp_c, _ = orc.quantize_w4_c(W)
    assert np.array_equal(wp, wp_c)


def test_quantize_w8_numpy_equals_c_and_closed_form():
    rng = np.random.default_rng(6)
    for name, W in _w_modes(rng, 5, 384):
        wq_n, s_n = orc.quantize_w8(W)
        wq_c, s_c = orc.quantize_w8_c(W)
        assert np.array_equal(wq_n, wq_c), name
        assert np.array_equal(s_n, s_c), name
        W32 = W.astype(np.float32)
        s32 = (np.abs(W32).max(axis=1) / np.float32(127)).astype(np.float32)
        assert np.array_equal(s_n, s32)
        assert np.abs(wq_n.astype(np.int32)).max() <= 127
    Wz = np.zeros((2, 16), np.float16)
    wq, s = orc.quantize_w8(Wz)
    assert np.all(s == 0) and np.all(wq == 0)


# ------------------------------------------- the gate rejects mistakes

def _y_sequential(q, scale, x):
    """float32 sequential dequant-dot for an explicit (possibly wrong) q."""
    N, K = q.shape
    y = np.zeros(N, np.float32)
    for n in range(N):
        w = q[n].astype(np.float32) * np.repeat(scale[n].astype(np.float32), 128)
        y[n] = np.float32(np.sum(w * x.astype(np.float32), dtype=np.float32))
    return y.astype(np.float16)


def test_gate_accepts_oracle_reference_for_all_modes():
    rng = np.random.default_rng(21)
    for name, W in _w_modes(rng, 8, 1024):
        wp, s = orc.quantize_w4(W)
        for xs in (1.0, 1e-4, 10.0):
            x = (rng.standard_normal(1024) * xs).astype(np.float16)
            _, y16 = orc.ref_f32_w4(wp, s, x)
            assert orc.check_w4(y16, wp, s, x) <= 1.0, (name, xs)


def test_gate_rejects_planted_mistakes():
    rng = np.random.default_rng(22)
    W = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float16)
    wp, s = orc.quantize_w4(W)
    x = rng.standard_normal(1024).astype(np.float16)
    q = orc.unpack_w(wp)
    good = _y_sequential(q, s, x)
    assert orc.check_w4(good, wp, s, x) <= 1.0
    b = wp.astype(np.int32)
    mistakes = {}
    # low/high nibble swapped
    qs = q.copy()
    qs[:, 0::2], qs[:, 1::2] = q[:, 1::2], q[:, 0::2]
    mistakes["nibble_swap"] = qs
    # no sign extension (codes 8..15 read as +8..+15)
    qn = np.empty_like(q)
    qn[:, 0::2] = b & 0xF
    qn[:, 1::2] = b >> 4
    mistakes["no_sign_extension"] = qn
    # last term dropped
    qd = q.copy()
    qd[:, -1] = 0
    mistakes["dropped_term"] = qd
    for name, qm in mistakes.items():
        y = _y_sequential(qm, s, x)
        assert orc.check_w4(y, wp, s, x) > 1.0, name
    # wrong group index (scale of group g//2 instead of g)
    s_wrong = s[:, np.arange(s.shape[1]) // 2]
    y = _y_sequential(q, s_wrong, x)
    assert orc.check_w4(y, wp, s, x) > 1.0
    # rows shifted by one
    y = np.roll(good, 1)
    assert orc.check_w4(y, wp, s, x) > 1.0
    # transposed/permuted x chunk (first two 16-byte chunks of x swapped)
    xp = x.copy()
    xp[:32], xp[32:64] = x[32:64], x[:32]
    y = _y_sequential(q, s, xp)
    assert orc.check_w4(y, wp, s, x) > 1.0


# ------------------------------------------------ FP16 / FP32 GEMV oracle

def _fp_inputs(rng, N, K, dt, scales=(1e-6, 1.0, 300.0)):
    W = (rng.standard_normal((N, K)) * rng.choice(scales, (N, K))).astype(dt)
    x = (rng.standard_normal(K) * rng.choice(scales, K)).astype(dt)
    return W, x


@pytest.mark.parametrize("dt", [np.float16, np.float32])
@pytest.mark.parametrize("N,K", [(3, 1), (5, 37), (4, 129)])
def test_exact_gemv_matches_fractions(dt, N, K):
    rng = np.random.default_rng(N * 1000 + K)
    W, x = _fp_inputs(rng, N, K, dt)
    ex, S = orc.exact_gemv(W, x)
    for r in range(N):
        terms = [Fraction(float(W[r, k])) * Fraction(float(x[k])) for k in range(K)]
        assert float(sum(terms)) == ex[r]
        assert float(sum(abs(t) for t in terms)) == S[r]


def test_exact_gemv_closed_forms():
    rng = np.random.default_rng(5)
    for dt in (np.float16, np.float32):
        W = rng.standard_normal((6, 40)).astype(dt)
        for j in (0, 17, 39):                       # one-hot x picks a column
            x = np.zeros(40, dtype=dt)
            x[j] = 1
            ex, S = orc.exact_gemv(W, x)
            assert np.array_equal(ex, W[:, j].astype(np.float64))
            assert np.array_equal(S, np.abs(W[:, j]).astype(np.float64))
        ones = np.ones(40, dtype=dt)                # all-ones x sums the rows
        ex, _ = orc.exact_gemv(np.ones((2, 40), dtype=dt), ones)
        assert np.array_equal(ex, np.full(2, 40.0))
    # fp16 subnormal products stay exact (2^-24 * 2^-24 = 2^-48)
    t = np.array([[2.0 ** -24] * 8], dtype=np.float16)
    ex, _ = orc.exact_gemv(t, np.full(8, 2.0 ** -24, dtype=np.float16))
    assert ex[0] == 8 * 2.0 ** -48


def test_ulp32_matches_spacing():
    v = np.array([0.0, 1e-45, 1.0, 3.5, 1e30, -2.0, 65504.0], dtype=np.float32)
    assert np.array_equal(orc.ulp32(v), np.spacing(np.abs(v)).astype(np.float64))


def _spacing16(v: np.ndarray) -> np.ndarray:
    """fp16 grid spacing from numpy's own nextafter on the fp16 type: the
    gap from |v| rounded to fp16 to the next fp16 above it, and for the
    largest finite value (whose next value would overflow) the gap below
    it, 65504 - 65472 = 32."""
    a = np.abs(np.asarray(v, dtype=np.float64).astype(np.float16))
    with np.errstate(over="ignore"):        # 65504's next value is inf
        up = np.nextafter(a, np.float16(np.inf))
    gap = up.astype(np.float64) - a.astype(np.float64)
    top = a == np.float16(65504.0)
    below = np.nextafter(a, np.float16(0.0)).astype(np.float64)
    return np.where(top, a.astype(np.float64) - below, gap)


def test_ulp16_matches_spacing_on_all_fp16_values():
    """ulp16 (oracle restatement of cudalab/int4gemv_correctness.py:128-141)
    against an independent definition over all 65536 fp16 bit patterns:
    every finite value below 65504 gets np.spacing's fp16 gap, 65504 gets
    32, subnormals and zeros get 2^-24."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = bits.view(np.float16)
    fin = np.isfinite(v)
    vf = v[fin]
    got = orc.ulp16(vf.astype(np.float64))
    want = _spacing16(vf)
    assert np.array_equal(got, want)
    a = np.abs(vf.astype(np.float64))
    below_max = a < 65504.0
    assert np.array_equal(got[below_max],
                          np.spacing(np.abs(vf[below_max])).astype(np.float64))
    assert np.all(got[a == 65504.0] == 32.0)
    sub = a < 2.0 ** -14
    assert sub.sum() == 2 * 1024          # +-0 and the 1023 subnormals each side
    assert np.all(got[sub] == 2.0 ** -24)
    assert fin.sum() == 63488             # 65536 - 2 infinities - 2046 NaNs


def test_ulp16_rounds_to_fp16_before_measuring():
    # values that round into the next binade take that binade's spacing
    v = np.array([1.0 + 2.0 ** -12, 2.0 - 2.0 ** -13, 65519.0, 3e-8, -0.0])
    got = orc.ulp16(v)
    assert np.array_equal(got, _spacing16(v))
    assert list(got) == [2.0 ** -10, 2.0 ** -9, 32.0, 2.0 ** -24, 2.0 ** -24]


def test_ulp16_pin_rejects_planted_mistakes():
    """Plausible slips in the ulp formula fail the pin above (planted here on
    the CPU, in copies of the formula): a factor of two either way, ceil for
    floor, and the subnormal floor taken as 2^-14."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = bits.view(np.float16)
    vf = v[np.isfinite(v)]
    want = _spacing16(vf)
    a = np.abs(vf.astype(np.float64))
    tiny = 2.0 ** -14
    with np.errstate(divide="ignore"):
        lg = np.log2(np.maximum(a, tiny))
    mistakes = {
        "half": np.where(a >= tiny, 2.0 ** (np.floor(lg) - 11), 2.0 ** -24),
        "double": np.where(a >= tiny, 2.0 ** (np.floor(lg) - 9), 2.0 ** -24),
        "ceil": np.where(a >= tiny, 2.0 ** (np.ceil(lg) - 10), 2.0 ** -24),
        "sub_floor": np.where(a >= tiny, 2.0 ** (np.floor(lg) - 10), tiny),
    }
    for name, bad in mistakes.items():
        assert not np.array_equal(bad, want), name


@pytest.mark.parametrize("dt", [np.float16, np.float32])
def test_gemv_gate_accepts_cpu_gemv_and_rejects_planted_mistakes(dt):
    rng = np.random.default_rng(11)
    N, K = 64, 1024
    W = rng.standard_normal((N, K)).astype(dt)
    x = rng.standard_normal(K).astype(dt)
    ex, S = orc.exact_gemv(W, x)
    y = orc.gemv_cpu(W, x, threads=2)
    assert orc.arith_ratio_gemv(y, ex, S, K, dt).max() <= 1.0
    # a dropped term (the last column) is far outside the bound
    y_drop = (W[:, :-1].astype(np.float64) @ x[:-1].astype(np.float64)).astype(dt)
    assert orc.arith_ratio_gemv(y_drop, ex, S, K, dt).max() > 1.0
    # the transposed operand (W^T of a square block)
    Wsq = W[:, :N]
    exq, Sq = orc.exact_gemv(np.ascontiguousarray(Wsq), x[:N].copy())
    y_t = (Wsq.T.astype(np.float64) @ x[:N].astype(np.float64)).astype(dt)
    assert orc.arith_ratio_gemv(y_t, exq, Sq, N, dt).max() > 1.0
    if dt == np.float16:
        # accumulating in fp16 instead of FP32 breaks the bound
        acc = np.zeros(N, dtype=np.float16)
        for k in range(K):
            acc = (acc + W[:, k] * x[k]).astype(np.float16)
        assert orc.arith_ratio_gemv(acc, ex, S, K, dt).max() > 1.0
