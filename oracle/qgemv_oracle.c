/*
 * qgemv_oracle.c -- CPU restatement of the reference's weight-only
 * quantized GEMV path, used as the parity checker.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker or the timed CPU baseline; the product path never calls it.
 *
 * What each function restates (reference file:line):
 *   orc_unpack_bytes    cudalab/int4gemv_quantize.py:117-134 (unpack_w) and
 *                       kernels/int4gemv/int4gemv_common.h:141-149
 *   orc_int4_quantize   cudalab/int4gemv_quantize.py:61-114 (quantize_w,
 *                       pack_q)
 *   orc_q8_quantize     cudalab/qgemv_quantize.py:33-64
 *                       (both take `rcp`: the scale amax / qmax as torch
 *                       evaluates it for a GPU tensor, amax * fl(1/qmax),
 *                       instead of the CPU's correctly rounded division)
 *   orc_int4_exact      the fp64 "exact" and S_n of the accumulation bound,
 *                       cudalab/int4gemv_correctness.py:175-209, computed
 *                       here in exact integer arithmetic (one rounding)
 *   orc_q8_exact        cudalab/qgemv_correctness.py:152-180, likewise
 *   orc_int4_ref_f32    the FP32 reference dequantize_w(...) @ x.float()
 *                       (cudalab/int4gemv_correctness.py:220-221), summed
 *                       in sequential k order
 *   orc_q8_ref_f32      cudalab/qgemv_correctness.py:189-190, likewise
 *   orc_int4_gemv_cpu   the same FP32 computation as a fused, row-parallel
 *   orc_q8_gemv_cpu     CPU kernel (OpenMP), for the CPU baseline timing
 *   orc_gemv_exact      the fp64 "exact" and S_n of the FP16/FP32 GEMV
 *                       bound (cudalab/gemv_correctness.py:175-200): fp16
 *                       in exact integer arithmetic (one rounding), fp32
 *                       as exact products summed in double-double
 *                       (relative error ~ K * 2^-106, far below the bound)
 *   orc_gemv_cpu        FP16/FP32 GEMV, FP32 accumulation, row-parallel
 *                       (OpenMP), the reference's gemv_ref formulation
 *                       torch.mv(W.float(), x.float()) (operators/gemv.py:
 *                       192-200) for the CPU baseline timing
 *
 * Exact arithmetic: every fp16 value is an integer multiple of 2^-24 with
 * magnitude below 2^40 (in units of 2^-24).  An INT4 term q*s*x is then an
 * integer times 2^-48 below 2^83, and a row sum over K <= 2^20 terms fits in
 * a signed 128-bit integer; converting that integer to double rounds once.
 * For INT8 the fp32 scale is an integer (24-bit significand) times a power
 * of two, and s * sum(q * x) is formed the same way.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef __int128 i128;

/* fp16 bits -> (integer m, so that value = m * 2^-24); returns 0 for inf/nan */
static int h_fixed(uint16_t h, int64_t* m) {
    const int sign = h >> 15;
    const int e = (h >> 10) & 0x1f;
    const int64_t f = h & 0x3ff;
    int64_t v;
    if (e == 0x1f) return 0;
    if (e == 0) v = f;                         /* subnormal: f * 2^-24 */
    else v = (1024 + f) << (e - 1);            /* (1024+f) * 2^(e-25) */
    *m = sign ? -v : v;
    return 1;
}

double orc_h2d(uint16_t h) {
    const int sign = h >> 15;
    const int e = (h >> 10) & 0x1f;
    const int f = h & 0x3ff;
    double v;
    if (e == 0x1f) v = f ? NAN : INFINITY;
    else if (e == 0) v = ldexp((double)f, -24);
    else v = ldexp((double)(1024 + f), e - 25);
    return sign ? -v : v;
}

/* float32 -> fp16 bits, round to nearest even, subnormals and overflow. */
uint16_t orc_f2h(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* >= 65520 */
    if (a < 0x38800000u) {                                    /* < 2^-14 */
        float mag;
        memcpy(&mag, &a, sizeof mag);
        /* exact product in double; nearbyint rounds half to even */
        const double q = nearbyint((double)mag * 16777216.0);  /* * 2^24 */
        return (uint16_t)(sign | (uint32_t)q);                 /* 1024 -> min normal */
    }
    uint32_t h = ((a >> 23) - 112u) << 10 | ((a & 0x7fffffu) >> 13);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

static float h2f(uint16_t h) { return (float)orc_h2d(h); }

static void unpack_byte(uint8_t b, int* lo, int* hi) {
    *lo = (b & 0x0f) - ((b & 0x08) << 1);
    *hi = (b >> 4) - ((b & 0x80) >> 3);
}

void orc_unpack_bytes(const uint8_t* b, int64_t nbytes, int32_t* out) {
    for (int64_t i = 0; i < nbytes; ++i) {
        int lo, hi;
        unpack_byte(b[i], &lo, &hi);
        out[2 * i] = lo;
        out[2 * i + 1] = hi;
    }
}

/* Exact row sums: exact[n] = sum_k q*s*x, S[n] = sum_k |q*s*x| (each one
 * rounding to double).  Returns 0, or -1 if an input holds inf/nan (then
 * the affected rows get NaN). */
int orc_int4_exact(const uint8_t* wp, const uint16_t* scale, const uint16_t* x,
                   int64_t n, int64_t k, double* exact, double* S) {
    const int64_t kb = k / 2, ng = k / 128;
    int bad = 0;
    for (int64_t r = 0; r < n; ++r) {
        i128 sum = 0, abs_sum = 0;
        int row_bad = 0;
        for (int64_t b = 0; b < kb; ++b) {
            int64_t ms, mx0, mx1;
            if (!h_fixed(scale[r * ng + b / 64], &ms) ||
                !h_fixed(x[2 * b], &mx0) || !h_fixed(x[2 * b + 1], &mx1)) {
                row_bad = 1;
                continue;
            }
            int lo, hi;
            unpack_byte(wp[r * kb + b], &lo, &hi);
            const i128 t0 = (i128)lo * ms * mx0;
            const i128 t1 = (i128)hi * ms * mx1;
            sum += t0 + t1;
            abs_sum += (t0 < 0 ? -t0 : t0) + (t1 < 0 ? -t1 : t1);
        }
        if (row_bad) {
            exact[r] = NAN;
            S[r] = NAN;
            bad = 1;
        } else {
            exact[r] = ldexp((double)sum, -48);
            S[r] = ldexp((double)abs_sum, -48);
        }
    }
    return bad ? -1 : 0;
}

int orc_q8_exact(const int8_t* wq, const float* scale, const uint16_t* x,
                 int64_t n, int64_t k, double* exact, double* S) {
    int bad = 0;
    for (int64_t r = 0; r < n; ++r) {
        const float s = scale[r];
        if (!isfinite(s)) {
            exact[r] = NAN;
            S[r] = NAN;
            bad = 1;
            continue;
        }
        int es = 0;
        const float fs = frexpf(s, &es);               /* s = fs * 2^es */
        const int64_t ms = (int64_t)ldexpf(fs, 24);    /* exact: 24-bit significand */
        i128 sum = 0, abs_sum = 0;
        int row_bad = 0;
        for (int64_t i = 0; i < k; ++i) {
            int64_t mx;
            if (!h_fixed(x[i], &mx)) { row_bad = 1; continue; }
            const i128 t = (i128)wq[r * k + i] * mx;
            sum += t;
            abs_sum += t < 0 ? -t : t;
        }
        if (row_bad) {
            exact[r] = NAN;
            S[r] = NAN;
            bad = 1;
            continue;
        }
        /* value = ms * sum * 2^(es - 24) * 2^-24 */
        const int64_t ams = ms < 0 ? -ms : ms;
        exact[r] = ldexp((double)(sum * ms), es - 48);
        S[r] = ldexp((double)(abs_sum * ams), es - 48);
    }
    return bad ? -1 : 0;
}

/* FP32 reference, sequential k: acc = acc + (q*s)*x with separate roundings
 * (q*s is exact in FP32), then one RNE cast to fp16. */
void orc_int4_ref_f32(const uint8_t* wp, const uint16_t* scale, const uint16_t* x,
                      int64_t n, int64_t k, float* y32, uint16_t* y16) {
    const int64_t kb = k / 2, ng = k / 128;
    for (int64_t r = 0; r < n; ++r) {
        float acc = 0.f;
        for (int64_t b = 0; b < kb; ++b) {
            const float s = h2f(scale[r * ng + b / 64]);
            int lo, hi;
            unpack_byte(wp[r * kb + b], &lo, &hi);
            const float w0 = (float)lo * s, w1 = (float)hi * s;
            const float p0 = w0 * h2f(x[2 * b]);
            acc = acc + p0;
            const float p1 = w1 * h2f(x[2 * b + 1]);
            acc = acc + p1;
        }
        if (y32) y32[r] = acc;
        if (y16) y16[r] = orc_f2h(acc);
    }
}

void orc_q8_ref_f32(const int8_t* wq, const float* scale, const uint16_t* x,
                    int64_t n, int64_t k, float* y32, uint16_t* y16) {
    for (int64_t r = 0; r < n; ++r) {
        const float s = scale[r];
        float acc = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            const float w = (float)wq[r * k + i] * s;
            const float p = w * h2f(x[i]);
            acc = acc + p;
        }
        if (y32) y32[r] = acc;
        if (y16) y16[r] = orc_f2h(acc);
    }
}

/* Symmetric group-wise INT4 quantizer: per group of 128, s32 = amax / 7 in
 * FP32; q = clamp(rint(w / s32), -7, 7) (ties to even); zero group -> s = 0,
 * q = 0; pack element 2b low nibble, 2b+1 high nibble; scale stored as
 * fp16(s32). */
void orc_int4_quantize(const uint16_t* w16, int64_t n, int64_t k, uint8_t* wp,
                       uint16_t* scale16, int rcp) {
    const float inv7 = 1.0f / 7.0f;
    const int64_t ng = k / 128;
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t g = 0; g < ng; ++g) {
            const uint16_t* src = w16 + r * k + g * 128;
            float amax = 0.f;
            for (int i = 0; i < 128; ++i) {
                const float a = fabsf(h2f(src[i]));
                if (a > amax) amax = a;
            }
            const float s32 = rcp ? amax * inv7 : amax / 7.0f;
            uint8_t* dst = wp + r * (k / 2) + g * 64;
            for (int i = 0; i < 64; ++i) {
                int q[2];
                for (int h = 0; h < 2; ++h) {
                    if (s32 == 0.f) { q[h] = 0; continue; }
                    float v = nearbyintf(h2f(src[2 * i + h]) / s32);
                    if (v > 7.f) v = 7.f;
                    if (v < -7.f) v = -7.f;
                    q[h] = (int)v;
                }
                dst[i] = (uint8_t)((q[0] & 0xf) | ((q[1] & 0xf) << 4));
            }
            scale16[r * ng + g] = orc_f2h(s32);
        }
    }
}

void orc_q8_quantize(const uint16_t* w16, int64_t n, int64_t k, int8_t* wq,
                     float* scale, int rcp) {
    const float inv127 = 1.0f / 127.0f;
    for (int64_t r = 0; r < n; ++r) {
        float amax = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            const float a = fabsf(h2f(w16[r * k + i]));
            if (a > amax) amax = a;
        }
        const float s = rcp ? amax * inv127 : amax / 127.0f;
        for (int64_t i = 0; i < k; ++i) {
            if (s == 0.f) { wq[r * k + i] = 0; continue; }
            float v = nearbyintf(h2f(w16[r * k + i]) / s);
            if (v > 127.f) v = 127.f;
            if (v < -127.f) v = -127.f;
            wq[r * k + i] = (int8_t)v;
        }
        scale[r] = s;
    }
}

/* ------------------------------------------------------- CPU baseline ---
 * Fused unpack -> dequant -> dot, rows in parallel (OpenMP), FP32
 * accumulation in 16 independent partial sums (a legal FP32 order under
 * the same bound), x converted to FP32 once per call into `xf` (caller
 * buffer of k floats). */
#define ORC_LANES 16

void orc_int4_gemv_cpu(const uint8_t* wp, const uint16_t* scale, const uint16_t* x,
                       uint16_t* y, int64_t n, int64_t k, int threads, float* xf) {
    const int64_t kb = k / 2, ng = k / 128;
    for (int64_t i = 0; i < k; ++i) xf[i] = h2f(x[i]);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        float acc[ORC_LANES] = {0};
        const uint8_t* row = wp + r * kb;
        for (int64_t g = 0; g < ng; ++g) {
            const float s = h2f(scale[r * ng + g]);
            const uint8_t* gb = row + g * 64;
            const float* gx = xf + g * 128;
            for (int i = 0; i < 64; i += ORC_LANES / 2) {
                for (int l = 0; l < ORC_LANES / 2; ++l) {
                    const uint8_t b = gb[i + l];
                    const float lo = (float)((b & 0x0f) - ((b & 0x08) << 1));
                    const float hi = (float)((b >> 4) - ((b & 0x80) >> 3));
                    acc[2 * l] = acc[2 * l] + (lo * s) * gx[2 * (i + l)];
                    acc[2 * l + 1] = acc[2 * l + 1] + (hi * s) * gx[2 * (i + l) + 1];
                }
            }
        }
        float t = 0.f;
        for (int l = 0; l < ORC_LANES; ++l) t = t + acc[l];
        y[r] = orc_f2h(t);
    }
}

void orc_q8_gemv_cpu(const int8_t* wq, const float* scale, const uint16_t* x,
                     uint16_t* y, int64_t n, int64_t k, int threads, float* xf) {
    for (int64_t i = 0; i < k; ++i) xf[i] = h2f(x[i]);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        float acc[ORC_LANES] = {0};
        const int8_t* row = wq + r * k;
        int64_t i = 0;
        for (; i + ORC_LANES <= k; i += ORC_LANES)
            for (int l = 0; l < ORC_LANES; ++l)
                acc[l] = acc[l] + (float)row[i + l] * xf[i + l];
        for (; i < k; ++i) acc[0] = acc[0] + (float)row[i] * xf[i];
        float t = 0.f;
        for (int l = 0; l < ORC_LANES; ++l) t = t + acc[l];
        y[r] = orc_f2h(scale[r] * t);
    }
}

/* ---- FP16 / FP32 GEMV ---------------------------------------------- */

/* Error-free sum a + b = s + e (Knuth's TwoSum). */
static void two_sum(double a, double b, double* s, double* e) {
    const double t = a + b;
    const double bb = t - a;
    *e = (a - (t - bb)) + (b - bb);
    *s = t;
}

/* dtype 0: w, x fp16 bits; dtype 1: w, x float32.  exact[n] = sum_k w*x,
 * S[n] = sum_k |w*x|.  Returns 0, or -1 if an input is inf/nan (then the
 * affected rows get NaN). */
int orc_gemv_exact(int dtype, const void* w, const void* x, int64_t n,
                   int64_t k, double* exact, double* S) {
    int bad = 0;
    if (dtype == 0) {
        const uint16_t* wh = (const uint16_t*)w;
        const uint16_t* xh = (const uint16_t*)x;
        for (int64_t r = 0; r < n; ++r) {
            i128 sum = 0, abs_sum = 0;
            int row_bad = 0;
            for (int64_t i = 0; i < k; ++i) {
                int64_t mw, mx;
                if (!h_fixed(wh[r * k + i], &mw) || !h_fixed(xh[i], &mx)) {
                    row_bad = 1;
                    continue;
                }
                const i128 t = (i128)mw * (i128)mx;   /* value * 2^48 */
                sum += t;
                abs_sum += t < 0 ? -t : t;
            }
            if (row_bad) {
                exact[r] = S[r] = NAN;
                bad = 1;
                continue;
            }
            exact[r] = ldexp((double)sum, -48);
            S[r] = ldexp((double)abs_sum, -48);
        }
        return bad ? -1 : 0;
    }
    const float* wf = (const float*)w;
    const float* xf = (const float*)x;
    for (int64_t r = 0; r < n; ++r) {
        double hi = 0.0, lo = 0.0, ahi = 0.0, alo = 0.0;
        int row_bad = 0;
        for (int64_t i = 0; i < k; ++i) {
            const float a = wf[r * k + i], b = xf[i];
            if (!isfinite(a) || !isfinite(b)) {
                row_bad = 1;
                continue;
            }
            const double t = (double)a * (double)b;   /* exact: 24 + 24 bits */
            double s1, e1;
            two_sum(hi, t, &s1, &e1);
            hi = s1;
            lo += e1;
            two_sum(ahi, fabs(t), &s1, &e1);
            ahi = s1;
            alo += e1;
        }
        if (row_bad) {
            exact[r] = S[r] = NAN;
            bad = 1;
            continue;
        }
        exact[r] = hi + lo;
        S[r] = ahi + alo;
    }
    return bad ? -1 : 0;
}

void orc_gemv_cpu(int dtype, const void* w, const void* x, void* y, int64_t n,
                  int64_t k, int threads, float* xf) {
    const uint16_t* wh = (const uint16_t*)w;
    const float* wf = (const float*)w;
    for (int64_t i = 0; i < k; ++i)
        xf[i] = dtype == 0 ? h2f(((const uint16_t*)x)[i]) : ((const float*)x)[i];
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        float acc[ORC_LANES] = {0};
        int64_t i = 0;
        if (dtype == 0) {
            const uint16_t* row = wh + r * k;
            for (; i + ORC_LANES <= k; i += ORC_LANES)
                for (int l = 0; l < ORC_LANES; ++l)
                    acc[l] = acc[l] + h2f(row[i + l]) * xf[i + l];
            for (; i < k; ++i) acc[0] = acc[0] + h2f(row[i]) * xf[i];
        } else {
            const float* row = wf + r * k;
            for (; i + ORC_LANES <= k; i += ORC_LANES)
                for (int l = 0; l < ORC_LANES; ++l)
                    acc[l] = acc[l] + row[i + l] * xf[i + l];
            for (; i < k; ++i) acc[0] = acc[0] + row[i] * xf[i];
        }
        float t = 0.f;
        for (int l = 0; l < ORC_LANES; ++l) t = t + acc[l];
        if (dtype == 0) ((uint16_t*)y)[r] = orc_f2h(t);
        else ((float*)y)[r] = t;
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
