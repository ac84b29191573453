"""CPU oracle of the weight-only quantized GEMV path (numpy + the C library
built from oracle/qgemv_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this module, and only as the checker
(or as the timed CPU baseline).  The product (cudalab_amd) never imports it.

Each function names the reference code it restates (paths are relative to
the reference repository).  How each is pinned (tests/test_oracle_*.py):
  unpack_w / pack_q       exhaustive 256-byte closed form and bijection
                          (tests/test_int4gemv_cpu.py:53-108 of the reference)
  quantize_w4 / _w8       closed-form invariants (scale == fp16(amax/7),
                          q == clamp(rint(W/s32)), zero groups, step bound,
                          half-even ties) and numpy == C == cudalab_amd;
                          the `rcp` scale form against a float64 restatement
                          of fl(amax * fl(1/qmax)) over every fp16 amax
  exact_w4 / exact_w8     exact rational arithmetic (fractions.Fraction) on
                          small inputs, one-hot and all-ones closed forms
  ref_f32_w4 / _w8        sequential FP32 sum replayed in numpy float32
  arith_ratio             the bound of cudalab/int4gemv_correctness.py:
                          175-209; planted mistakes (nibble swap, lost sign
                          extension, wrong group, dropped term) exceed it
  exact_gemv              Fraction arithmetic on small fp16/fp32 inputs,
                          one-hot and constant closed forms
  arith_ratio_gemv        the bound of cudalab/gemv_correctness.py:175-200;
                          planted mistakes (transposed W, dropped term,
                          fp16 accumulation) exceed it
  ulp32                   numpy.spacing on float32
  expect_exact_*          the exact value cast once to the output type, for
                          inputs whose every FP32 partial sum is exact in any
                          order (conditions checked on entry); pinned against
                          exact_* and Fraction sums (tests/test_exact_inputs_cpu.py)
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_qgemv.so"
GROUP_SIZE = 128
INT4_MAX = 7
INT8_MAX = 127
TOL_K = 2.0
PER_TERM_ROUNDINGS = 3.0

_lib = None


def build() -> Path:
    """Compile the C oracle (make -B)."""
    subprocess.run(["make", "-B", "-C", str(HERE)], check=True,
                   stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_int4_exact.argtypes = [P, P, P, i64, i64, P, P]
        L.orc_int4_exact.restype = ctypes.c_int
        L.orc_q8_exact.argtypes = [P, P, P, i64, i64, P, P]
        L.orc_q8_exact.restype = ctypes.c_int
        L.orc_int4_ref_f32.argtypes = [P, P, P, i64, i64, P, P]
        L.orc_q8_ref_f32.argtypes = [P, P, P, i64, i64, P, P]
        L.orc_int4_quantize.argtypes = [P, i64, i64, P, P, ctypes.c_int]
        L.orc_q8_quantize.argtypes = [P, i64, i64, P, P, ctypes.c_int]
        L.orc_unpack_bytes.argtypes = [P, i64, P]
        L.orc_int4_gemv_cpu.argtypes = [P, P, P, P, i64, i64, ctypes.c_int, P]
        L.orc_q8_gemv_cpu.argtypes = [P, P, P, P, i64, i64, ctypes.c_int, P]
        L.orc_gemv_exact.argtypes = [ctypes.c_int, P, P, i64, i64, P, P]
        L.orc_gemv_exact.restype = ctypes.c_int
        L.orc_gemv_cpu.argtypes = [ctypes.c_int, P, P, P, i64, i64, ctypes.c_int, P]
        L.orc_f2h.argtypes = [ctypes.c_float]
        L.orc_f2h.restype = ctypes.c_uint16
        L.orc_h2d.argtypes = [ctypes.c_uint16]
        L.orc_h2d.restype = ctypes.c_double
        L.orc_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _bits16(a: np.ndarray) -> np.ndarray:
    """fp16 array -> its uint16 bit patterns (contiguous)."""
    return np.ascontiguousarray(np.asarray(a, dtype=np.float16)).view(np.uint16)


# ------------------------------------------------------- packing (numpy)

def unpack_w(wp: np.ndarray) -> np.ndarray:
    """uint8 (N, K/2) -> int32 (N, K), 4-bit two's complement, element 2b
    from the low nibble (cudalab/int4gemv_quantize.py:117-134)."""
    wp = np.asarray(wp, dtype=np.uint8)
    b = wp.astype(np.int32)
    lo = (b & 0xF) - ((b & 0x8) << 1)
    hi = (b >> 4) - ((b & 0x80) >> 3)
    out = np.empty((wp.shape[0], 2 * wp.shape[1]), dtype=np.int32)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def pack_q(q: np.ndarray) -> np.ndarray:
    """int (N, K) in [-8, 7], K even -> uint8 (N, K/2)
    (cudalab/int4gemv_quantize.py:92-114)."""
    q = np.asarray(q, dtype=np.int64)
    if q.ndim != 2 or q.shape[1] % 2:
        raise ValueError("pack_q needs (N, K) with K even")
    if q.size and (q.min() < -8 or q.max() > 7):
        raise ValueError("pack_q: values outside [-8, 7]")
    lo = q[:, 0::2] & 0xF
    hi = q[:, 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_w_c(wp: np.ndarray) -> np.ndarray:
    """Same as unpack_w, through the C restatement."""
    wp = np.ascontiguousarray(wp, dtype=np.uint8)
    out = np.empty((wp.shape[0], 2 * wp.shape[1]), dtype=np.int32)
    lib().orc_unpack_bytes(_p(wp), wp.size, _p(out))
    return out


# ----------------------------------------------------- quantizers (numpy)

def _scale(amax: np.ndarray, qmax: int, rcp: bool) -> np.ndarray:
    """amax / qmax in FP32 as torch evaluates `tensor / python_int`: one
    correctly rounded division for a CPU tensor; for a GPU tensor a product
    with the FP32 reciprocal fl(1/qmax), rounded once (torch turns a CPU
    scalar divisor into a multiplication by its reciprocal: PyTorch
    aten/src/ATen/native/cuda/BinaryDivTrueKernel.cu, div_true_kernel_cuda)."""
    amax = amax.astype(np.float32)
    if rcp:
        inv = np.float32(1) / np.float32(qmax)
        return (amax * inv).astype(np.float32)
    return (amax / np.float32(qmax)).astype(np.float32)


def quantize_w4(W16: np.ndarray, rcp: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Group-wise INT4 (cudalab/int4gemv_quantize.py:61-89): FP32 amax/7
    (see `_scale` for `rcp`), round half to even, clamp +-7, zero groups ->
    0; returns (uint8 packed, fp16 scale)."""
    W16 = np.asarray(W16, dtype=np.float16)
    N, K = W16.shape
    if K % GROUP_SIZE:
        raise ValueError("K % 128 != 0")
    g = W16.astype(np.float32).reshape(N, K // GROUP_SIZE, GROUP_SIZE)
    s32 = _scale(np.abs(g).max(axis=2), INT4_MAX, rcp)
    zero = s32 == 0
    denom = np.where(zero, np.float32(1), s32).astype(np.float32)
    q = np.rint((g / denom[:, :, None]).astype(np.float32))
    q = np.clip(q, -INT4_MAX, INT4_MAX)
    q[np.broadcast_to(zero[:, :, None], q.shape)] = 0
    return pack_q(q.reshape(N, K).astype(np.int64)), s32.astype(np.float16)


def quantize_w8(W16: np.ndarray, rcp: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Per-row INT8 (cudalab/qgemv_quantize.py:33-64): (int8 W_q, fp32
    scale); `rcp` as for quantize_w4."""
    W32 = np.asarray(W16, dtype=np.float16).astype(np.float32)
    s = _scale(np.abs(W32).max(axis=1), INT8_MAX, rcp)
    zero = s == 0
    denom = np.where(zero, np.float32(1), s).astype(np.float32)
    q = np.rint((W32 / denom[:, None]).astype(np.float32))
    q = np.clip(q, -INT8_MAX, INT8_MAX)
    q[zero] = 0
    return q.astype(np.int8), s


def quantize_w4_c(W16: np.ndarray, rcp: bool = False) -> tuple[np.ndarray, np.ndarray]:
    Wb = _bits16(W16)
    N, K = Wb.shape
    wp = np.empty((N, K // 2), dtype=np.uint8)
    sc = np.empty((N, K // GROUP_SIZE), dtype=np.uint16)
    lib().orc_int4_quantize(_p(Wb), N, K, _p(wp), _p(sc), int(rcp))
    return wp, sc.view(np.float16)


def quantize_w8_c(W16: np.ndarray, rcp: bool = False) -> tuple[np.ndarray, np.ndarray]:
    Wb = _bits16(W16)
    N, K = Wb.shape
    wq = np.empty((N, K), dtype=np.int8)
    sc = np.empty((N,), dtype=np.float32)
    lib().orc_q8_quantize(_p(Wb), N, K, _p(wq), _p(sc), int(rcp))
    return wq, sc


def dequantize_w4(wp: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """FP32 q * fp16 scale (cudalab/int4gemv_quantize.py:137-149)."""
    q = unpack_w(wp)
    s = np.repeat(np.asarray(scale, dtype=np.float16).astype(np.float32),
                  GROUP_SIZE, axis=1)
    return q.astype(np.float32) * s


# ------------------------------------------------- exact values (C, int128)

def exact_w4(wp: np.ndarray, scale: np.ndarray, x: np.ndarray):
    """(exact, S) per row, each rounded once to double from an exact
    integer sum."""
    wp = np.ascontiguousarray(wp, dtype=np.uint8)
    sb, xb = _bits16(scale), _bits16(x)
    N, K = wp.shape[0], 2 * wp.shape[1]
    ex = np.empty(N, dtype=np.float64)
    S = np.empty(N, dtype=np.float64)
    lib().orc_int4_exact(_p(wp), _p(sb), _p(xb), N, K, _p(ex), _p(S))
    return ex, S


def exact_w8(wq: np.ndarray, scale: np.ndarray, x: np.ndarray):
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    sc = np.ascontiguousarray(scale, dtype=np.float32)
    xb = _bits16(x)
    N, K = wq.shape
    ex = np.empty(N, dtype=np.float64)
    S = np.empty(N, dtype=np.float64)
    lib().orc_q8_exact(_p(wq), _p(sc), _p(xb), N, K, _p(ex), _p(S))
    return ex, S


def ref_f32_w4(wp, scale, x):
    """Sequential-k FP32 reference; returns (y32 float32, y16 float16)."""
    wp = np.ascontiguousarray(wp, dtype=np.uint8)
    sb, xb = _bits16(scale), _bits16(x)
    N, K = wp.shape[0], 2 * wp.shape[1]
    y32 = np.empty(N, dtype=np.float32)
    y16 = np.empty(N, dtype=np.uint16)
    lib().orc_int4_ref_f32(_p(wp), _p(sb), _p(xb), N, K, _p(y32), _p(y16))
    return y32, y16.view(np.float16)


def ref_f32_w8(wq, scale, x):
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    sc = np.ascontiguousarray(scale, dtype=np.float32)
    xb = _bits16(x)
    N, K = wq.shape
    y32 = np.empty(N, dtype=np.float32)
    y16 = np.empty(N, dtype=np.uint16)
    lib().orc_q8_ref_f32(_p(wq), _p(sc), _p(xb), N, K, _p(y32), _p(y16))
    return y32, y16.view(np.float16)


# ------------------------------------------------------------- the gate

def ulp16(v: np.ndarray) -> np.ndarray:
    """fp16 grid spacing at |v| (2^-24 below the smallest normal)."""
    a = np.abs(np.asarray(v, dtype=np.float64).astype(np.float16)
               .astype(np.float64))
    tiny = 2.0 ** -14
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.maximum(a, tiny)))
    return np.where(a >= tiny, np.power(2.0, e - 10), 2.0 ** -24)


def arith_ratio(y16: np.ndarray, exact: np.ndarray, S: np.ndarray,
                K: int) -> np.ndarray:
    """Per-row |y - exact| / tol with
    tol = TOL_K * (3*K*2^-24*S + ulp16(y)/2 + ulp16(exact)/2)
    (cudalab/int4gemv_correctness.py:175-209); non-finite -> inf."""
    y = np.asarray(y16, dtype=np.float16).astype(np.float64)
    tol = TOL_K * (PER_TERM_ROUNDINGS * K * 2.0 ** -24 * S
                   + 0.5 * ulp16(y) + 0.5 * ulp16(exact))
    diff = np.abs(y - exact)
    with np.errstate(invalid="ignore"):
        r = diff / tol
    return np.where(np.isfinite(r), r, np.inf)


# ------------------------------------------------ FP16 / FP32 GEMV

def _gemv_dtype(a: np.ndarray) -> int:
    if a.dtype == np.float16:
        return 0
    if a.dtype == np.float32:
        return 1
    raise TypeError(f"gemv oracle takes float16 or float32, got {a.dtype}")


def exact_gemv(W: np.ndarray, x: np.ndarray):
    """(exact, S) per row of the FP16/FP32 GEMV W @ x: fp16 in exact
    integer arithmetic, fp32 as exact products in double-double."""
    W = np.ascontiguousarray(W)
    x = np.ascontiguousarray(x)
    dt = _gemv_dtype(W)
    if x.dtype != W.dtype:
        raise TypeError("x and W must share a dtype")
    N, K = W.shape
    ex = np.empty(N, dtype=np.float64)
    S = np.empty(N, dtype=np.float64)
    lib().orc_gemv_exact(dt, _p(W), _p(x), N, K, _p(ex), _p(S))
    return ex, S


def ulp32(v: np.ndarray) -> np.ndarray:
    """float32 grid spacing at |v| (nextafter toward +inf minus v, as
    cudalab/gemv_correctness.py:_ulp does for float32)."""
    a = np.abs(np.asarray(v, dtype=np.float64).astype(np.float32))
    with np.errstate(over="ignore", invalid="ignore"):
        return (np.nextafter(a, np.float32(np.inf)) - a).astype(np.float64)


GEMV_TERM_ROUNDINGS = 2.0


def arith_ratio_gemv(y: np.ndarray, exact: np.ndarray, S: np.ndarray,
                     K: int, dtype) -> np.ndarray:
    """Per-row |y - exact| / tol with
    tol = TOL_K * (2*K*2^-24*S + ulp(y)/2 + ulp(exact)/2) on the grid of
    `dtype` (cudalab/gemv_correctness.py:175-200); non-finite -> inf."""
    dt = np.dtype(dtype)
    ulp = ulp16 if dt == np.float16 else ulp32
    yd = np.asarray(y).astype(dt).astype(np.float64)
    tol = TOL_K * (GEMV_TERM_ROUNDINGS * K * 2.0 ** -24 * S
                   + 0.5 * ulp(yd) + 0.5 * ulp(exact))
    diff = np.abs(yd - exact)
    with np.errstate(invalid="ignore"):
        r = diff / tol
    return np.where(np.isfinite(r), r, np.inf)


def check_gemv(y, W, x) -> float:
    ex, S = exact_gemv(W, x)
    r = arith_ratio_gemv(y, ex, S, np.asarray(W).shape[1], np.asarray(W).dtype)
    return float(r.max()) if r.size else 0.0


def gemv_cpu(W: np.ndarray, x: np.ndarray, threads: int | None = None) -> np.ndarray:
    """Fused OpenMP CPU FP16/FP32 GEMV, FP32 accumulation."""
    W = np.ascontiguousarray(W)
    x = np.ascontiguousarray(x)
    dt = _gemv_dtype(W)
    N, K = W.shape
    y = np.empty(N, dtype=W.dtype)
    xf = np.empty(K, dtype=np.float32)
    lib().orc_gemv_cpu(dt, _p(W), _p(x), _p(y), N, K, threads or max_threads(), _p(xf))
    return y


def check_w4(y16, wp, scale, x) -> float:
    """Max bound ratio of a kernel output against the oracle (<= 1 passes)."""
    ex, S = exact_w4(wp, scale, x)
    r = arith_ratio(y16, ex, S, 2 * np.asarray(wp).shape[1])
    return float(r.max()) if r.size else 0.0


def check_w8(y16, wq, scale, x) -> float:
    ex, S = exact_w8(wq, scale, x)
    r = arith_ratio(y16, ex, S, np.asarray(wq).shape[1])
    return float(r.max()) if r.size else 0.0


# ------------------------------------------------------- CPU baseline

def gemv_w4_cpu(wp, scale, x, threads: int | None = None) -> np.ndarray:
    """Fused OpenMP CPU GEMV (the timed CPU baseline)."""
    wp = np.ascontiguousarray(wp, dtype=np.uint8)
    sb, xb = _bits16(scale), _bits16(x)
    N, K = wp.shape[0], 2 * wp.shape[1]
    y = np.empty(N, dtype=np.uint16)
    xf = np.empty(K, dtype=np.float32)
    t = threads or max_threads()
    lib().orc_int4_gemv_cpu(_p(wp), _p(sb), _p(xb), _p(y), N, K, t, _p(xf))
    return y.view(np.float16)


def gemv_w8_cpu(wq, scale, x, threads: int | None = None) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    sc = np.ascontiguousarray(scale, dtype=np.float32)
    xb = _bits16(x)
    N, K = wq.shape
    y = np.empty(N, dtype=np.uint16)
    xf = np.empty(K, dtype=np.float32)
    t = threads or max_threads()
    lib().orc_q8_gemv_cpu(_p(wq), _p(sc), _p(xb), _p(y), N, K, t, _p(xf))
    return y.view(np.float16)


def max_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        return int(env)
    return int(lib().orc_max_threads())


# ------------------------------------------- exact-input expectations
#
# For inputs built so that every FP32 partial sum of the products is exact
# whatever the summation order, the only rounding left in any correct kernel
# is the final cast of the exact value to the output type.  Its result is
# then known bit for bit, at any K and for every variant (the fixed bound
# above allows 6K roundings per term, so at large K it cannot see a dropped
# chunk of work; this can).
#
# INT4: scales are powers of two in [2^-6, 2^-2], x in {-1, 0, +1}, and
#   K <= 131072.  Every product q * s * x is a multiple of 2^-6 with
#   |q * s| <= 2, so every partial sum is a multiple of 2^-6 of magnitude
#   at most 2K <= 2^18: at most 2^24 units of 2^-6, exact in FP32.
# INT8: scales are powers of two in [2^-8, 2^0] (one per row), x in
#   {-1, 0, +1}, K <= 131072.  Per row the partial sums are s times an
#   integer of magnitude at most 128K <= 2^24: exact, applied before or
#   after the scale.
# FP16/FP32: every W element is q * 2^-e with q an integer, |q| <= 8 and
#   e in [2, 6], x in {-1, 0, +1}, K <= 131072: multiples of 2^-6 below
#   2^18, as for INT4.

EXACT_MAX_K = 131072


def _pow2_exponents(v: np.ndarray) -> np.ndarray:
    m, e = np.frexp(np.asarray(v, dtype=np.float64))
    if np.any(m != 0.5):
        raise ValueError("exact-input condition: every scale must be a power of two")
    return e - 1


def _unit_x(x: np.ndarray) -> None:
    xf = np.asarray(x).astype(np.float64)
    if not np.all(np.isin(xf, (-1.0, 0.0, 1.0))):
        raise ValueError("exact-input condition: x must lie in {-1, 0, +1}")


def expect_exact_w4(wp: np.ndarray, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """fp16 of the exact INT4 GEMV for exact inputs (conditions above)."""
    K = 2 * np.asarray(wp).shape[1]
    if K > EXACT_MAX_K:
        raise ValueError(f"exact-input condition: K = {K} > {EXACT_MAX_K}")
    e = _pow2_exponents(np.asarray(scale, dtype=np.float16))
    if e.size and (e.min() < -6 or e.max() > -2):
        raise ValueError("exact-input condition: INT4 scales in [2^-6, 2^-2]")
    _unit_x(x)
    ex, _ = exact_w4(wp, scale, x)
    return ex.astype(np.float16)


def expect_exact_w8(wq: np.ndarray, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """fp16 of the exact INT8 GEMV for exact inputs (conditions above)."""
    K = np.asarray(wq).shape[1]
    if K > EXACT_MAX_K:
        raise ValueError(f"exact-input condition: K = {K} > {EXACT_MAX_K}")
    e = _pow2_exponents(np.asarray(scale, dtype=np.float32))
    if e.size and (e.min() < -8 or e.max() > 0):
        raise ValueError("exact-input condition: INT8 scales in [2^-8, 1]")
    _unit_x(x)
    ex, _ = exact_w8(wq, scale, x)
    return ex.astype(np.float16)


def expect_exact_gemv(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The exact FP16/FP32 GEMV cast to W's dtype, for exact inputs."""
    W = np.asarray(W)
    K = W.shape[1]
    if K > EXACT_MAX_K:
        raise ValueError(f"exact-input condition: K = {K} > {EXACT_MAX_K}")
    w = W.astype(np.float64)
    u = w * 64.0                              # in units of 2^-6
    if np.any(u != np.round(u)) or np.any(np.abs(w) > 2.0):
        raise ValueError("exact-input condition: W must be multiples of 2^-6 "
                         "of magnitude at most 2")
    _unit_x(x)
    ex, _ = exact_gemv(W, np.asarray(x, dtype=W.dtype))
    return ex.astype(W.dtype)
