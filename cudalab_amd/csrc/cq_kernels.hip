// gfx950 (CDNA4) kernels of the weight-only quantized GEMV path, plus their
// launch-shape selection.
//
// Semantics follow the reference operator contracts
// (kernels/int4gemv/int4gemv_common.h:1-79 for INT4,
//  kernels/qgemv/qgemv_common.h:1-55 for INT8): FP32 accumulation, one
// round-to-nearest-even cast to fp16 per output row, fp16 subnormals kept
// (the library is never built with fast-math or flush-to-zero).
//
// Two kernel families per operator:
//
// * scalar (`*_scalar_kernel`): one 256-thread workgroup per row, strided
//   1-byte weight loads, per-element dequant `fma(q*s, x, acc)`, DPP wave
//   reduction, LDS across the 4 waves.  It has no alignment requirement and
//   is the single source for the *_baseline variants and for every
//   fallback (bit-identity of fallback and baseline follows from that).
//
// * wave (`*_wave_kernel<CW, J, R>`): the CDNA4 design.
//   - Lanes of a wave64 are split into 64/CW row slots of CW lanes; lane
//     (slot, col) owns the 16-byte weight chunks col, col+CW, ...,
//     col+CW*(J-1) of every row it handles, so one wave load instruction
//     reads CW*16 contiguous bytes of each of 64/CW rows (fully coalesced).
//   - Each lane handles R rows; all R*J weight loads are issued before any
//     arithmetic, so a whole row tile is in flight at once (HBM latency is
//     the limiter for these short kernels).
//   - The lane's x values for its J chunks are loaded once and kept in
//     registers as fp16 pairs, reused across its R rows.
//   - Nibbles become fp16 with one v_bitop3 per pair:
//       ((w & 0x000F000F) ^ 0x64086408) is the fp16 pair (1032+q0, 1032+q4)
//     (4-bit two's complement q, xor 8 maps it to q+8, 0x6400 is 1024), and
//     one packed fp16 add of -1032 gives (q0, q4) exactly.  The nibbles at
//     bits 4-7 are taken in place as 16*q ((w & 0x00F000F0) ^ 0x64806480,
//     bias -1152) and their partial sum is scaled by 1/16 (exact).
//   - Products and sums use v_dot2_f32_f16 (fp16 x fp16 products are exact
//     in FP32, accumulation in FP32); the group scale is applied once per
//     16-byte chunk (one chunk lies inside one 128-element group).
//   - Cross-lane reduction uses DPP (quad_perm, row mirrors, row_bcast15/31)
//     with no LDS and no barrier; the last lane of each row segment writes.
//   INT8 uses the same structure with 16 int8 per chunk:
//       ((w & 0x00FF00FF) ^ 0x64806480) - 1152 = (q0, q2) as fp16,
//   and the per-row scale applied once after the reduction.
//
// Every wave-kernel summation order is a legal FP32 order under the
// reference's accumulation-error bound (at most three FP32 roundings per
// term: the dot2 rounding, the scale product, the accumulate).

#include "cq_internal.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <type_traits>

namespace cq {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kBlock = 256;  // threads per workgroup for every kernel

__device__ __forceinline__ float h2f(uint16_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ uint16_t f2h(float v) {
    // v_cvt_f16_f32: round to nearest even, fp16 subnormals kept.
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

__device__ __forceinline__ f16x2 as_f16x2(uint32_t bits) {
    return __builtin_bit_cast(f16x2, bits);
}

// v + (v moved by a DPP pattern).  Lanes of rows outside ROW_MASK receive
// +0, which leaves their value unchanged.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_plus(float v) {
    const int moved = __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false);
    return v + __builtin_bit_cast(float, moved);
}

// Sum over aligned segments of SEG lanes (16, 32 or 64).  The total is
// exact in the last lane of every segment (lane % SEG == SEG - 1).
template <int SEG>
__device__ __forceinline__ float segment_sum(float v) {
    v = dpp_plus<0xB1>(v);   // quad_perm [1,0,3,2]: pairs
    v = dpp_plus<0x4E>(v);   // quad_perm [2,3,0,1]: quads
    v = dpp_plus<0x141>(v);  // row_half_mirror: 8 lanes
    v = dpp_plus<0x140>(v);  // row_mirror: 16 lanes
    if constexpr (SEG >= 32) v = dpp_plus<0x142, 0xA>(v);  // row_bcast15
    if constexpr (SEG >= 64) v = dpp_plus<0x143, 0xC>(v);  // row_bcast31
    return v;
}

// ---------------------------------------------------------------- scalar

__global__ __launch_bounds__(kBlock) void int4gemv_scalar_kernel(
        const uint8_t* __restrict__ w, const uint16_t* __restrict__ scale,
        const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
        int64_t k) {
    const int64_t row = blockIdx.x;
    const int64_t kb = k >> 1;  // bytes per row
    const uint8_t* __restrict__ wrow = w + row * kb;
    const uint16_t* __restrict__ srow = scale + row * (k >> 7);
    float acc = 0.f;
    for (int64_t b = threadIdx.x; b < kb; b += kBlock) {
        const uint32_t byte = wrow[b];
        const float s = h2f(srow[b >> 6]);  // both nibbles: group b/64
        // sign-extend bits 0-3 (element 2b) and bits 4-7 (element 2b+1)
        const int32_t lo = static_cast<int32_t>(byte << 28) >> 28;
        const int32_t hi = static_cast<int32_t>(byte << 24) >> 28;
        acc = __builtin_fmaf(static_cast<float>(lo) * s, h2f(x[2 * b]), acc);
        acc = __builtin_fmaf(static_cast<float>(hi) * s, h2f(x[2 * b + 1]),
                             acc);
    }
    acc = segment_sum<64>(acc);
    __shared__ float part[kBlock / 64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 63) part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) y[row] = f2h((part[0] + part[1]) + (part[2] + part[3]));
}

__global__ __launch_bounds__(kBlock) void qgemv_scalar_kernel(
        const int8_t* __restrict__ w, const float* __restrict__ scale,
        const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
        int64_t k) {
    const int64_t row = blockIdx.x;
    const int8_t* __restrict__ wrow = w + row * k;
    const float s = scale[row];
    float acc = 0.f;
    for (int64_t i = threadIdx.x; i < k; i += kBlock)
        acc = __builtin_fmaf(static_cast<float>(wrow[i]) * s, h2f(x[i]), acc);
    acc = segment_sum<64>(acc);
    __shared__ float part[kBlock / 64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 63) part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) y[row] = f2h((part[0] + part[1]) + (part[2] + part[3]));
}

// ------------------------------------------------------------------ wave

// Rows per lane that the register budget of a J-chunk instance allows.
constexpr int int4_rmax(int j) { return j <= 2 ? 4 : (j <= 4 ? 2 : 1); }
constexpr int q8_rmax(int j) { return j <= 4 ? 4 : (j <= 8 ? 2 : 1); }
constexpr int kInt4MaxJ = 8;   // 8 * 64 chunks * 32 = 16384 elements
constexpr int kQ8MaxJ = 16;    // 16 * 64 chunks * 16 = 16384 elements

template <int CW, int J, int R>
__global__ __launch_bounds__(kBlock) void int4gemv_wave_kernel(
        const uint4* __restrict__ w,         // [n][nchunks] 16-byte chunks
        const uint16_t* __restrict__ scale,  // [n][nchunks/4]
        const uint4* __restrict__ x,         // [nchunks][4] 16-byte pieces
        uint16_t* __restrict__ y, int n, int nchunks) {
    constexpr int SLOTS = 64 / CW;
    const int lane = threadIdx.x & 63;
    const int col = lane % CW;
    const int slot = lane / CW;
    const int ngroups = nchunks >> 2;
    const int64_t wave_id =
        static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t row0 = wave_id * (SLOTS * R) + slot;

    // Every load is unconditional on a clamped, in-bounds index (lanes past
    // the row end or past n re-read a valid chunk) so that no load sits
    // behind a branch and all of them are in flight together; inactive
    // lanes are zeroed afterwards with a select.  Weight chunks of all R
    // rows go first: the HBM requests leave at once.
    int cidx[J];
    bool act[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = col + CW * j;
        act[j] = c < nchunks;
        cidx[j] = act[j] ? c : nchunks - 1;
    }
    uint4 wv[R][J];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = std::min<int64_t>(row0 + SLOTS * r, n - 1);
#pragma unroll
        for (int j = 0; j < J; ++j) wv[r][j] = w[row * nchunks + cidx[j]];
    }
    uint16_t sv[R][J];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = std::min<int64_t>(row0 + SLOTS * r, n - 1);
#pragma unroll
        for (int j = 0; j < J; ++j) sv[r][j] = scale[row * ngroups + (cidx[j] >> 2)];
    }
    uint4 xv[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int p = 0; p < 4; ++p) xv[j][p] = x[4 * cidx[j] + p];

    // x of the lane's chunks, re-paired for the nibble order of a weight
    // word: xa = (x0,x4), xb = (x1,x5), xc = (x2,x6), xd = (x3,x7).  An
    // inactive chunk gets x = 0, so its (valid, re-read) weights add +-0.
    uint32_t xa[J][4], xb[J][4], xc[J][4], xd[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        uint32_t d[16];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            d[4 * p + 0] = act[j] ? xv[j][p].x : 0u;
            d[4 * p + 1] = act[j] ? xv[j][p].y : 0u;
            d[4 * p + 2] = act[j] ? xv[j][p].z : 0u;
            d[4 * p + 3] = act[j] ? xv[j][p].w : 0u;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t d0 = d[4 * q], d1 = d[4 * q + 1];
            const uint32_t d2 = d[4 * q + 2], d3 = d[4 * q + 3];
            xa[j][q] = (d0 & 0xFFFFu) | (d2 << 16);
            xb[j][q] = (d0 >> 16) | (d2 & 0xFFFF0000u);
            xc[j][q] = (d1 & 0xFFFFu) | (d3 << 16);
            xd[j][q] = (d1 >> 16) | (d3 & 0xFFFF0000u);
        }
    }

    const f16x2 bias1 = {static_cast<_Float16>(-1032.0f),
                         static_cast<_Float16>(-1032.0f)};
    const f16x2 bias16 = {static_cast<_Float16>(-1152.0f),
                          static_cast<_Float16>(-1152.0f)};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t words[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z,
                                       wv[r][j].w};
            float d1 = 0.f, d16 = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t u = words[q];
                const uint32_t u8 = u >> 8;
                const f16x2 qa = as_f16x2((u & 0x000F000Fu) ^ 0x64086408u) + bias1;
                const f16x2 qb = as_f16x2((u & 0x00F000F0u) ^ 0x64806480u) + bias16;
                const f16x2 qc = as_f16x2((u8 & 0x000F000Fu) ^ 0x64086408u) + bias1;
                const f16x2 qd = as_f16x2((u8 & 0x00F000F0u) ^ 0x64806480u) + bias16;
                d1 = __builtin_amdgcn_fdot2(qa, as_f16x2(xa[j][q]), d1, false);
                d16 = __builtin_amdgcn_fdot2(qb, as_f16x2(xb[j][q]), d16, false);
                d1 = __builtin_amdgcn_fdot2(qc, as_f16x2(xc[j][q]), d1, false);
                d16 = __builtin_amdgcn_fdot2(qd, as_f16x2(xd[j][q]), d16, false);
            }
            const float s = h2f(sv[r][j]);
            acc = __builtin_fmaf(s, d1, acc);
            acc = __builtin_fmaf(s * 0.0625f, d16, acc);
        }
        acc = segment_sum<CW>(acc);
        const int64_t row = row0 + SLOTS * r;
        if (col == CW - 1 && row < n) y[row] = f2h(acc);
    }
}

template <int CW, int J, int R>
__global__ __launch_bounds__(kBlock) void qgemv_wave_kernel(
        const uint4* __restrict__ w,       // [n][nchunks] 16 int8 per chunk
        const float* __restrict__ scale,   // [n]
        const uint4* __restrict__ x,       // [nchunks][2] 16-byte pieces
        uint16_t* __restrict__ y, int n, int nchunks) {
    constexpr int SLOTS = 64 / CW;
    const int lane = threadIdx.x & 63;
    const int col = lane % CW;
    const int slot = lane / CW;
    const int64_t wave_id =
        static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t row0 = wave_id * (SLOTS * R) + slot;

    // Unconditional loads on clamped indices, as in the INT4 kernel.
    int cidx[J];
    bool act[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = col + CW * j;
        act[j] = c < nchunks;
        cidx[j] = act[j] ? c : nchunks - 1;
    }
    uint4 wv[R][J];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = std::min<int64_t>(row0 + SLOTS * r, n - 1);
#pragma unroll
        for (int j = 0; j < J; ++j) wv[r][j] = w[row * nchunks + cidx[j]];
    }
    uint4 xv[J][2];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        xv[j][0] = x[2 * cidx[j]];
        xv[j][1] = x[2 * cidx[j] + 1];
    }
    // x re-paired for a weight word's byte order: xp = (x0,x2), xq = (x1,x3);
    // an inactive chunk gets x = 0.
    uint32_t xp[J][4], xq[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint4 v0 = xv[j][0], v1 = xv[j][1];
        uint32_t d[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = act[j] ? d[i] : 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t d0 = d[2 * q], d1 = d[2 * q + 1];
            xp[j][q] = (d0 & 0xFFFFu) | (d1 << 16);
            xq[j][q] = (d0 >> 16) | (d1 & 0xFFFF0000u);
        }
    }

    const f16x2 bias = {static_cast<_Float16>(-1152.0f),
                        static_cast<_Float16>(-1152.0f)};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t words[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z,
                                       wv[r][j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t u = words[q];
                const f16x2 qp = as_f16x2((u & 0x00FF00FFu) ^ 0x64806480u) + bias;
                const f16x2 qq = as_f16x2(((u >> 8) & 0x00FF00FFu) ^ 0x64806480u) + bias;
                acc = __builtin_amdgcn_fdot2(qp, as_f16x2(xp[j][q]), acc, false);
                acc = __builtin_amdgcn_fdot2(qq, as_f16x2(xq[j][q]), acc, false);
            }
        }
        acc = segment_sum<CW>(acc);
        const int64_t row = row0 + SLOTS * r;
        if (col == CW - 1 && row < n) y[row] = f2h(scale[row] * acc);
    }
}

// --------------------------------------------------------- instance tables

using Int4WaveFn = void (*)(const uint4*, const uint16_t*, const uint4*,
                            uint16_t*, int, int);
using Q8WaveFn = void (*)(const uint4*, const float*, const uint4*,
                          uint16_t*, int, int);

template <int CW, int J, int R>
constexpr Int4WaveFn int4_instance() {
    if constexpr (R <= int4_rmax(J)) return &int4gemv_wave_kernel<CW, J, R>;
    else return nullptr;
}
template <int CW, int J, int R>
constexpr Q8WaveFn q8_instance() {
    if constexpr (R <= q8_rmax(J)) return &qgemv_wave_kernel<CW, J, R>;
    else return nullptr;
}

constexpr int r_index(int r) { return r == 1 ? 0 : (r == 2 ? 1 : 2); }

template <int CW, int J>
Int4WaveFn int4_pick_r(int r) {
    static constexpr Int4WaveFn t[3] = {int4_instance<CW, J, 1>(),
                                        int4_instance<CW, J, 2>(),
                                        int4_instance<CW, J, 4>()};
    return t[r_index(r)];
}
template <int CW, int J>
Q8WaveFn q8_pick_r(int r) {
    static constexpr Q8WaveFn t[3] = {q8_instance<CW, J, 1>(),
                                      q8_instance<CW, J, 2>(),
                                      q8_instance<CW, J, 4>()};
    return t[r_index(r)];
}

template <int... Js>
Int4WaveFn int4_pick_j64(int j, int r, std::integer_sequence<int, Js...>) {
    Int4WaveFn f = nullptr;
    ((j == Js + 1 ? (f = int4_pick_r<64, Js + 1>(r), 0) : 0), ...);
    return f;
}
template <int... Js>
Q8WaveFn q8_pick_j64(int j, int r, std::integer_sequence<int, Js...>) {
    Q8WaveFn f = nullptr;
    ((j == Js + 1 ? (f = q8_pick_r<64, Js + 1>(r), 0) : 0), ...);
    return f;
}

Int4WaveFn int4_wave_fn(int cw, int j, int r) {
    if (cw == 16 && j == 1) return int4_pick_r<16, 1>(r);
    if (cw == 32 && j == 1) return int4_pick_r<32, 1>(r);
    if (cw == 64 && j >= 1 && j <= kInt4MaxJ)
        return int4_pick_j64(j, r, std::make_integer_sequence<int, kInt4MaxJ>{});
    return nullptr;
}
Q8WaveFn q8_wave_fn(int cw, int j, int r) {
    if (cw == 16 && j == 1) return q8_pick_r<16, 1>(r);
    if (cw == 32 && j == 1) return q8_pick_r<32, 1>(r);
    if (cw == 64 && j >= 1 && j <= kQ8MaxJ)
        return q8_pick_j64(j, r, std::make_integer_sequence<int, kQ8MaxJ>{});
    return nullptr;
}

// Launch with the argument types taken from the kernel's own signature.
template <typename... Params>
hipError_t launch(void (*kernel)(Params...), int64_t grid, int block,
                  hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1,
                  std::type_identity_t<Params>... args) {
    void* argv[] = {static_cast<void*>(&args)...};
    const dim3 g(static_cast<uint32_t>(grid)), b(static_cast<uint32_t>(block));
    if (ev0 == nullptr && ev1 == nullptr)
        return hipLaunchKernel(reinterpret_cast<const void*>(kernel), g, b,
                               argv, 0, stream);
    return hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), g, b,
                              argv, 0, stream, ev0, ev1, 0);
}

int pow2_at_least(int64_t v, int lo) {
    int p = lo;
    while (p < v && p < 64) p <<= 1;
    return p;
}

// Default rows per lane: the largest R the instance allows that still gives
// at least `min_waves` waves (8 per CU on a 256-CU part), so the chip is
// filled and every SIMD holds more than one wave.
int default_rows(int64_t n, int slots, int rmax) {
    constexpr int64_t min_waves = 2048;
    for (int r = rmax; r > 1; r >>= 1) {
        const int64_t waves = (n + slots * r - 1) / (slots * r);
        if (waves >= min_waves) return r;
    }
    return 1;
}

void finish_wave_plan(Plan& p, int64_t n) {
    const int slots = 64 / p.cw;
    const int64_t rows_per_wave = static_cast<int64_t>(slots) * p.r;
    const int64_t waves = (n + rows_per_wave - 1) / rows_per_wave;
    const int64_t block_waves = std::min<int64_t>(kBlock / 64, waves);
    p.block = static_cast<int>(block_waves * 64);
    p.grid = (waves + block_waves - 1) / block_waves;
}

Plan scalar_plan(int64_t n, bool fallback, const char* why) {
    Plan p;
    p.kind = kScalar;
    p.block = kBlock;
    p.grid = n;
    p.fallback = fallback;
    p.why = why;
    return p;
}

}  // namespace

bool int4_contract_ok(const void* w, const void* x, int64_t k) {
    if (k % 32 != 0) return false;
    return (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

bool q8_contract_ok(const void* w, const void* x, int64_t k) {
    if (k % 16 != 0) return false;
    return (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

Plan plan_int4(int kind, int rows, int64_t n, int64_t k, const void* w,
               const void* x) {
    if (kind == kScalar) return scalar_plan(n, false, "");
    if (!int4_contract_ok(w, x, k))
        return scalar_plan(n, true, "vector contract unmet (w/x 16B alignment, k%32)");
    if (k > kMaxWaveK) return scalar_plan(n, true, "k above the wave kernels' register-resident x");
    const int64_t nchunks = k / 32;
    Plan p;
    p.kind = kWave;
    p.cw = pow2_at_least(nchunks, 16);
    p.j = static_cast<int>((nchunks + p.cw - 1) / p.cw);
    const int rmax = int4_rmax(p.j);
    p.r = rows > 0 ? std::min(rows, rmax) : default_rows(n, 64 / p.cw, rmax);
    if (p.r == 3) p.r = 2;
    finish_wave_plan(p, n);
    return p;
}

Plan plan_q8(int kind, int rows, int64_t n, int64_t k, const void* w,
             const void* x) {
    if (kind == kScalar) return scalar_plan(n, false, "");
    if (!q8_contract_ok(w, x, k))
        return scalar_plan(n, true, "vector contract unmet (w/x 16B alignment, k%16)");
    if (k > kMaxWaveK) return scalar_plan(n, true, "k above the wave kernels' register-resident x");
    const int64_t nchunks = k / 16;
    Plan p;
    p.kind = kWave;
    p.cw = pow2_at_least(nchunks, 16);
    p.j = static_cast<int>((nchunks + p.cw - 1) / p.cw);
    const int rmax = q8_rmax(p.j);
    p.r = rows > 0 ? std::min(rows, rmax) : default_rows(n, 64 / p.cw, rmax);
    if (p.r == 3) p.r = 2;
    finish_wave_plan(p, n);
    return p;
}

hipError_t launch_int4(const Plan& p, const void* w, const void* scale,
                       const void* x, void* y, int64_t n, int64_t k,
                       hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    if (p.kind == kScalar)
        return launch(int4gemv_scalar_kernel, p.grid, p.block, stream, ev0, ev1,
                      static_cast<const uint8_t*>(w),
                      static_cast<const uint16_t*>(scale),
                      static_cast<const uint16_t*>(x),
                      static_cast<uint16_t*>(y), k);
    const Int4WaveFn fn = int4_wave_fn(p.cw, p.j, p.r);
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    return launch(fn, p.grid, p.block, stream, ev0, ev1,
                  static_cast<const uint4*>(w),
                  static_cast<const uint16_t*>(scale),
                  static_cast<const uint4*>(x), static_cast<uint16_t*>(y),
                  static_cast<int>(n), static_cast<int>(k / 32));
}

hipError_t launch_q8(const Plan& p, const void* w, const void* scale,
                     const void* x, void* y, int64_t n, int64_t k,
                     hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    if (p.kind == kScalar)
        return launch(qgemv_scalar_kernel, p.grid, p.block, stream, ev0, ev1,
                      static_cast<const int8_t*>(w),
                      static_cast<const float*>(scale),
                      static_cast<const uint16_t*>(x),
                      static_cast<uint16_t*>(y), k);
    const Q8WaveFn fn = q8_wave_fn(p.cw, p.j, p.r);
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    return launch(fn, p.grid, p.block, stream, ev0, ev1,
                  static_cast<const uint4*>(w),
                  static_cast<const float*>(scale),
                  static_cast<const uint4*>(x), static_cast<uint16_t*>(y),
                  static_cast<int>(n), static_cast<int>(k / 16));
}

}  // namespace cq
