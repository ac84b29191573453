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
#include <climits>
#include <cstring>
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

// Workgroups of a launch are dealt round-robin to the 8 XCDs (workgroup i
// runs on XCD i % 8), and each XCD has its own L2.  This returns a logical
// block index under which every XCD owns one contiguous range of logical
// blocks, so each XCD streams one contiguous range of weight rows and
// writes one contiguous range of y.  It is a bijection on [0, gridDim.x)
// for any grid size, so it changes which workgroup computes a row, never
// how the row is computed (outputs are bit-identical to the identity
// mapping).  Measured on MI355X at the bench shapes: 1-5% faster for INT4
// and up to 16% for INT8 than the identity mapping.
__device__ __forceinline__ uint32_t xcd_contiguous_block() {
    constexpr uint32_t kXcds = 8;
    const uint32_t b = blockIdx.x, g = gridDim.x;
    const uint32_t q = g / kXcds, r = g % kXcds;
    const uint32_t xcd = b % kXcds, idx = b / kXcds;
    return xcd * q + (xcd < r ? xcd : r) + idx;
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

// ------------------------------------------------------------- wave+LDS
//
// Second CDNA4 design: x is staged once per workgroup in LDS, already
// re-paired for the weight words, instead of every wave loading and
// re-pairing its own copy.  Per lane the x pairs of its J chunks then come
// from 4*J ds_read_b128.  Both nibbles of a byte feed one accumulator: the
// high nibble is taken in place (bits 4-7) under the fp16 exponent of 64,
// where the mantissa step is 1/16, so ((w & 0x00F000F0) ^ 0x54805480) is
// the fp16 pair (72+q1, 72+q5) and a packed add of -72 gives (q1, q5)
// exactly.  Workgroups take their rows through xcd_contiguous_block(); NT
// (256 or 512 threads) is chosen by the host plan.
//
// Address work is kept off the VALU, which these kernels are short of (the
// INT4 dequant and dot take 13 VALU instructions per 8 weights):
// - The host plans J = ceil(nchunks / CW), so a lane's chunks col + CW*j for
//   j < J - 1 always lie inside the row; only the last one is clamped.
//   The others sit at compile-time offsets from one per-lane address.
// - The LDS planes have the compile-time stride CW*J + 1; column CW*J is
//   zero and is what lanes past the row end read.  Every x read but the
//   last chunk's is then an immediate offset from one address.
// - The row base is wave-uniform when a row spans the wave (CW = 64), so it
//   lives in scalar registers.
// Issue order, pinned with scheduling barriers: the workgroup's x pieces,
// then per row, chunk by chunk, the group scale and the weight chunk
// (INT8: the chunks, then the row scale), so that the wait before chunk j
// covers chunks 0..j only and each chunk is summed as it lands.  A
// scheduling barrier after the workgroup barrier keeps weight arithmetic
// (and its waits) from being hoisted above it.

// The timeline stamps pin their clock reads by data dependence, not by
// scheduling fences (the compiler places pure arithmetic before the machine
// scheduler sees a fence, and a full fence also held every LDS read of x
// live at once, doubling the VGPRs at J = 6).  wall_clock_through(v) reads
// the wall clock with `v` passed through as an operand it may modify: the
// read waits for the arithmetic that produces v, and whatever uses v after
// it waits for the read.  The read is a scalar memory instruction the
// compiler does not track, so it waits for its own result before anything
// else counts on the LGKM counter.
__device__ __forceinline__ uint64_t wall_clock_through(float& v) {
    uint64_t t;
    asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t), "+v"(v));
    return t;
}
__device__ __forceinline__ uint64_t wall_clock_through(uint32_t& a, uint32_t& b,
                                                       uint32_t& c) {
    uint64_t t;
    asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)"
                 : "=s"(t), "+v"(a), "+v"(b), "+v"(c));
    return t;
}

// The rows of logical workgroup `blk` of one INT4 problem.  `xs` is the
// workgroup's LDS: [4][CW*J + 1] re-paired x pieces, q-major.
//
// STAMP (the timeline diagnostic only; every GEMV instance has it false, and
// then none of its code exists): lane 0 of each wave writes 8 words to
// stamps[wave * 8 ..]: the 100 MHz wall clock at the wave's start, after the
// x barrier, after its first chunk is summed, after its last chunk is
// summed and after its y stores are issued; then the hardware CU id.
template <int CW, int J, int R, int NT, bool STAMP = false>
__device__ __forceinline__ void int4_lds_rows(
        const uint4* __restrict__ w,         // [n][nchunks] 16-byte chunks
        const uint16_t* __restrict__ scale,  // [n][nchunks/4]
        const uint4* __restrict__ x,         // [4*nchunks] 16-byte pieces
        uint16_t* __restrict__ y, int n, int nchunks, uint32_t blk,
        uint4* __restrict__ xs, uint64_t* __restrict__ stamps = nullptr) {
    [[maybe_unused]] uint64_t ts[5] = {};
    if constexpr (STAMP) ts[0] = wall_clock64();
    constexpr int SLOTS = 64 / CW;
    constexpr int S = CW * J + 1;                     // LDS plane stride
    constexpr int XPER = (4 * CW * J + NT - 1) / NT;  // x pieces per thread
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int col = lane % CW;
    const int slot = lane / CW;
    const int npieces = 4 * nchunks;
    const int64_t wave_id = static_cast<int64_t>(blk) * (NT >> 6) +
                            __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t row0 = wave_id * (SLOTS * R) + slot;
    // Byte offsets fit in 32 bits (the host checks n * k / 2 < 2^32).
    const char* wb = reinterpret_cast<const char*>(w);
    const char* sb = reinterpret_cast<const char*>(scale);
    const uint32_t wrow_bytes = static_cast<uint32_t>(nchunks) * 16u;
    const uint32_t srow_bytes = static_cast<uint32_t>(nchunks >> 2) * 2u;

    // (1) this thread's share of x first
    uint4 xv[XPER];
#pragma unroll
    for (int i = 0; i < XPER; ++i) xv[i] = x[std::min(tid + i * NT, npieces - 1)];
    __builtin_amdgcn_sched_barrier(0);
    // (2) per row, each chunk's group scale and then the chunk, all in
    //     flight together; a last chunk past the row end re-reads chunk
    //     nchunks - 1 (x is zero there)
    const int clast = col + CW * (J - 1);
    const int cl = clast < nchunks ? clast : nchunks - 1;
    const uint32_t wcol = static_cast<uint32_t>(col) * 16u;
    const uint32_t scol = static_cast<uint32_t>(col >> 2) * 2u;
    uint4 wv[R][J];
    uint16_t sv[R][J];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = static_cast<uint32_t>(std::min<int64_t>(row0 + SLOTS * r, n - 1));
        const char* wr = wb + row * wrow_bytes;
        const char* sr = sb + row * srow_bytes;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool in_row = j < J - 1;
            sv[r][j] = *reinterpret_cast<const uint16_t*>(
                sr + (in_row ? scol + (CW / 2) * j : static_cast<uint32_t>(cl >> 2) * 2u));
            __builtin_amdgcn_sched_barrier(0);
            wv[r][j] = *reinterpret_cast<const uint4*>(
                wr + (in_row ? wcol + CW * 16 * j : static_cast<uint32_t>(cl) * 16u));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // (3) re-pair x: piece = x0..x7 -> [(x0,x4), (x1,x5), (x2,x6), (x3,x7)]
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
        // unconditional store on the clamped index (threads past the end
        // rewrite the last piece with the same value), so that no load is
        // sunk behind a branch
        const int p = std::min(tid + i * NT, npieces - 1);
        const uint4 v = xv[i];
        uint4 o;
        o.x = (v.x & 0xFFFFu) | (v.z << 16);
        o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
        o.z = (v.y & 0xFFFFu) | (v.w << 16);
        o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
        xs[(p & 3) * S + (p >> 2)] = o;
    }
    if (tid < 4) xs[tid * S + CW * J] = uint4{0, 0, 0, 0};
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // nibble masks and byte shift of the dequant; the stamped copy passes
    // them through the barrier stamp's clock read, so no dequant (nor its
    // wait for the weights) is placed above that read
    uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, sh8 = 8;
    if constexpr (STAMP) ts[1] = wall_clock_through(m_lo, m_hi, sh8);
    uint4 xp[J][4];
    const int xlast = clast < nchunks ? clast : CW * J;
    // the stamped copy reads each chunk's x next to its use (below): its
    // clock reads keep loads from crossing them, and reads issued all up
    // front would hold J x 16 VGPRs at once
    if constexpr (!STAMP) {
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                xp[j][q] = xs[q * S + (j < J - 1 ? col + CW * j : xlast)];
    }

    const f16x2 bias_lo = {static_cast<_Float16>(-1032.0f),
                           static_cast<_Float16>(-1032.0f)};
    const f16x2 bias_hi = {static_cast<_Float16>(-72.0f),
                           static_cast<_Float16>(-72.0f)};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if constexpr (STAMP) {
                if (r == 0) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        xp[j][q] = xs[q * S + (j < J - 1 ? col + CW * j : xlast)];
                }
            }
            float d = 0.f;
            if constexpr (STAMP) {
                // the second chunk's dequant and sum start after the first stamp
                if (r * J + j == 1)
                    asm volatile("" : "+v"(d), "+v"(wv[r][j].x), "+v"(wv[r][j].y),
                                 "+v"(wv[r][j].z), "+v"(wv[r][j].w) : "v"(acc));
            }
            const uint32_t words[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z,
                                       wv[r][j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t u = words[q];
                const uint32_t u8 = u >> sh8;
                const f16x2 qa = as_f16x2((u & m_lo) ^ 0x64086408u) + bias_lo;
                const f16x2 qb = as_f16x2((u & m_hi) ^ 0x54805480u) + bias_hi;
                const f16x2 qc = as_f16x2((u8 & m_lo) ^ 0x64086408u) + bias_lo;
                const f16x2 qd = as_f16x2((u8 & m_hi) ^ 0x54805480u) + bias_hi;
                d = __builtin_amdgcn_fdot2(qa, as_f16x2(xp[j][q].x), d, false);
                d = __builtin_amdgcn_fdot2(qb, as_f16x2(xp[j][q].y), d, false);
                d = __builtin_amdgcn_fdot2(qc, as_f16x2(xp[j][q].z), d, false);
                d = __builtin_amdgcn_fdot2(qd, as_f16x2(xp[j][q].w), d, false);
            }
            acc = __builtin_fmaf(h2f(sv[r][j]), d, acc);
            if constexpr (STAMP) {
                if (r == 0 && j == 0) ts[2] = wall_clock_through(acc);
                if (r == R - 1 && j == J - 1) ts[3] = wall_clock_through(acc);
            }
        }
        acc = segment_sum<CW>(acc);
        const int64_t row = row0 + SLOTS * r;
        if (col == CW - 1 && row < n) y[row] = f2h(acc);
    }
    if constexpr (STAMP) {
        __builtin_amdgcn_sched_barrier(0);
        ts[4] = wall_clock64();
        if (lane == 0) {
            const uint64_t wave = static_cast<uint64_t>(blk) * (NT >> 6) +
                                  static_cast<uint64_t>(tid >> 6);
            uint64_t* o = stamps + wave * 8;
#pragma unroll
            for (int i = 0; i < 5; ++i) o[i] = ts[i];
            o[5] = __smid();
            o[6] = 0;
            o[7] = 0;
        }
    }
}

// The rows of logical workgroup `blk` of one INT8 problem; `xs` holds
// [2][CW*J + 1] re-paired x pieces, q-major, column CW*J zero.  Same
// layout and issue order as the INT4 rows; the row's scale is loaded right
// after its weights, so the final scaling waits on no load of its own.
template <int CW, int J, int R, int NT>
__device__ __forceinline__ void q8_lds_rows(
        const uint4* __restrict__ w,       // [n][nchunks] 16 int8 per chunk
        const float* __restrict__ scale,   // [n]
        const uint4* __restrict__ x,       // [2*nchunks] 16-byte pieces
        uint16_t* __restrict__ y, int n, int nchunks, uint32_t blk,
        uint4* __restrict__ xs) {
    constexpr int SLOTS = 64 / CW;
    constexpr int S = CW * J + 1;
    constexpr int XPER = (2 * CW * J + NT - 1) / NT;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int col = lane % CW;
    const int slot = lane / CW;
    const int npieces = 2 * nchunks;
    const int64_t wave_id = static_cast<int64_t>(blk) * (NT >> 6) +
                            __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t row0 = wave_id * (SLOTS * R) + slot;
    const char* wb = reinterpret_cast<const char*>(w);
    const uint32_t wrow_bytes = static_cast<uint32_t>(nchunks) * 16u;

    uint4 xv[XPER];
#pragma unroll
    for (int i = 0; i < XPER; ++i) xv[i] = x[std::min(tid + i * NT, npieces - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const int clast = col + CW * (J - 1);
    const int cl = clast < nchunks ? clast : nchunks - 1;
    const uint32_t wcol = static_cast<uint32_t>(col) * 16u;
    uint4 wv[R][J];
    float sc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = static_cast<uint32_t>(std::min<int64_t>(row0 + SLOTS * r, n - 1));
        const char* wr = wb + row * wrow_bytes;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t off = j < J - 1 ? wcol + CW * 16 * j
                                           : static_cast<uint32_t>(cl) * 16u;
            wv[r][j] = *reinterpret_cast<const uint4*>(wr + off);
            __builtin_amdgcn_sched_barrier(0);
        }
        sc[r] = scale[row];
        __builtin_amdgcn_sched_barrier(0);
    }
    // re-pair x: piece = x0..x7 -> [(x0,x2), (x1,x3), (x4,x6), (x5,x7)]
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
        const int p = std::min(tid + i * NT, npieces - 1);
        const uint4 v = xv[i];
        uint4 o;
        o.x = (v.x & 0xFFFFu) | (v.y << 16);
        o.y = (v.x >> 16) | (v.y & 0xFFFF0000u);
        o.z = (v.z & 0xFFFFu) | (v.w << 16);
        o.w = (v.z >> 16) | (v.w & 0xFFFF0000u);
        xs[(p & 1) * S + (p >> 1)] = o;
    }
    if (tid < 2) xs[tid * S + CW * J] = uint4{0, 0, 0, 0};
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    uint4 xp[J][2];
    const int xlast = clast < nchunks ? clast : CW * J;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q)
            xp[j][q] = xs[q * S + (j < J - 1 ? col + CW * j : xlast)];

    const f16x2 bias = {static_cast<_Float16>(-1152.0f),
                        static_cast<_Float16>(-1152.0f)};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t words[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z,
                                       wv[r][j].w};
            const uint32_t xpair[8] = {xp[j][0].x, xp[j][0].y, xp[j][0].z,
                                       xp[j][0].w, xp[j][1].x, xp[j][1].y,
                                       xp[j][1].z, xp[j][1].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t u = words[q];
                const f16x2 qp = as_f16x2((u & 0x00FF00FFu) ^ 0x64806480u) + bias;
                const f16x2 qq = as_f16x2(((u >> 8) & 0x00FF00FFu) ^ 0x64806480u) + bias;
                acc = __builtin_amdgcn_fdot2(qp, as_f16x2(xpair[2 * q]), acc, false);
                acc = __builtin_amdgcn_fdot2(qq, as_f16x2(xpair[2 * q + 1]), acc, false);
            }
        }
        acc = segment_sum<CW>(acc);
        const int64_t row = row0 + SLOTS * r;
        if (col == CW - 1 && row < n) y[row] = f2h(sc[r] * acc);
    }
}

// LDS bytes of the untiled INT4 / INT8 LDS kernels for plan (cw, j).
constexpr uint32_t int4_lds_bytes(int cw, int j) {
    return 4u * 16u * static_cast<uint32_t>(cw * j + 1);
}
constexpr uint32_t q8_lds_bytes(int cw, int j) {
    return 2u * 16u * static_cast<uint32_t>(cw * j + 1);
}
// The LDS kernels read chunks col + cw*j for j < J - 1 unclamped, which
// stays inside a row only when J = ceil(nchunks / cw); every plan has that
// form, and launches check it.
inline bool lds_chunks_ok(const Plan& p, int64_t nchunks) {
    return p.cw > 0 && p.j == (nchunks + p.cw - 1) / p.cw;
}

// One problem per launch.
template <int CW, int J, int R, int NT>
__global__ __launch_bounds__(NT) void int4gemv_lds_kernel(
        const uint4* __restrict__ w, const uint16_t* __restrict__ scale,
        const uint4* __restrict__ x, uint16_t* __restrict__ y, int n,
        int nchunks) {
    extern __shared__ uint4 xs[];
    int4_lds_rows<CW, J, R, NT>(w, scale, x, y, n, nchunks,
                                xcd_contiguous_block(), xs);
}

// The INT4 LDS kernel with the timeline stamps (diagnostic, cq_int4_timeline):
// the same arithmetic and launch shape; `stamps` holds 8 words per wave.
template <int CW, int J, int R, int NT>
__global__ __launch_bounds__(NT) void int4gemv_lds_stamp_kernel(
        const uint4* __restrict__ w, const uint16_t* __restrict__ scale,
        const uint4* __restrict__ x, uint16_t* __restrict__ y, int n,
        int nchunks, uint64_t* __restrict__ stamps) {
    extern __shared__ uint4 xs[];
    int4_lds_rows<CW, J, R, NT, true>(w, scale, x, y, n, nchunks,
                                      xcd_contiguous_block(), xs, stamps);
}

template <int CW, int J, int R, int NT>
__global__ __launch_bounds__(NT) void qgemv_lds_kernel(
        const uint4* __restrict__ w, const float* __restrict__ scale,
        const uint4* __restrict__ x, uint16_t* __restrict__ y, int n,
        int nchunks) {
    extern __shared__ uint4 xs[];
    q8_lds_rows<CW, J, R, NT>(w, scale, x, y, n, nchunks,
                              xcd_contiguous_block(), xs);
}

// K-tiled LDS kernels, for rows longer than one batch of chunks held per
// lane (k > 16384; the *_lds_tiled variants force them at any k).  R rows
// per wave (CW = 64), both read against one copy of x.  x is staged tile by
// tile: TJ * 64 chunks of the row per tile (TJ = 2..8: TJ * 2048 INT4 or
// TJ * 1024 INT8 elements), re-paired in LDS, with a barrier before the
// tile is read and one before the next tile overwrites it.  Every thread of the workgroup
// runs the same tiles (they depend on nchunks only; rows past n are
// clamped, never skipped), so every barrier is reached by all.  In the last,
// partial tile only the first ceil(tc / 64) chunks of each lane are loaded
// and summed (a wave-uniform bound).  Lane `col` takes chunks col + 64 j of
// its rows in j order, as the untiled kernels do, so each row's sum
// accumulates in the same order as an untiled kernel with J =
// ceil(nchunks / 64): at k <= 16384 the result is bit-identical to the LDS
// kernel with CW = 64 (for any R).
template <int NT, int TJ, int R>
__global__ __launch_bounds__(NT) void int4gemv_tiled_kernel(
        const uint4* __restrict__ w, const uint16_t* __restrict__ scale,
        const uint4* __restrict__ x, uint16_t* __restrict__ y, int n,
        int nchunks) {
    extern __shared__ uint4 xs[];                  // [4][TC + 1]
    constexpr int TC = TJ * 64;                    // chunks per tile
    constexpr int XPER = 4 * TC / NT;              // x pieces per thread per tile
    static_assert(4 * TC % NT == 0, "a tile's pieces divide over the workgroup");
    constexpr int ldsw = TC + 1;
    const int tid = threadIdx.x;
    const int col = tid & 63;
    const int64_t row0 = (static_cast<int64_t>(xcd_contiguous_block()) * (NT >> 6) + (tid >> 6)) * R;
    // Byte offsets within a row fit in 32 bits (the host checks
    // n * k / 2 < 2^32); row bases are 64-bit.
    const char* wrow[R];
    const char* srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint64_t rc = static_cast<uint64_t>(std::min<int64_t>(row0 + r, n - 1));
        wrow[r] = reinterpret_cast<const char*>(w) + rc * (static_cast<uint32_t>(nchunks) * 16u);
        srow[r] = reinterpret_cast<const char*>(scale) + rc * ((static_cast<uint32_t>(nchunks) >> 2) * 2u);
    }
    const f16x2 bias_lo = {static_cast<_Float16>(-1032.0f),
                           static_cast<_Float16>(-1032.0f)};
    const f16x2 bias_hi = {static_cast<_Float16>(-72.0f),
                           static_cast<_Float16>(-72.0f)};
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    auto tile = [&]<bool PARTIAL>(int c0, int tc) {
        const int jn = PARTIAL ? (tc + 63) >> 6 : TJ;   // chunks per lane, wave-uniform
        const int np = 4 * tc;                          // x pieces in this tile
        const uint4* xt = x + 4 * static_cast<int64_t>(c0);
        uint4 xv[XPER];
#pragma unroll
        for (int i = 0; i < XPER; ++i) xv[i] = xt[std::min(tid + i * NT, np - 1)];
        __builtin_amdgcn_sched_barrier(0);
        // this lane's chunks of the tile; lanes past the row end re-read the
        // tile's last chunk against the zero column of x
        uint4 wv[R][TJ];
        uint16_t sv[R][TJ];
        int xcol[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            if (PARTIAL && j >= jn) break;
            const int c = col + 64 * j;
            const uint32_t cl = static_cast<uint32_t>(c0 + (c < tc ? c : tc - 1));
            xcol[j] = c < tc ? c : TC;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wv[r][j] = *reinterpret_cast<const uint4*>(wrow[r] + cl * 16u);
                sv[r][j] = *reinterpret_cast<const uint16_t*>(srow[r] + (cl >> 2) * 2u);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < XPER; ++i) {
            const int p = std::min(tid + i * NT, np - 1);
            const uint4 v = xv[i];
            uint4 o;
            o.x = (v.x & 0xFFFFu) | (v.z << 16);
            o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
            o.z = (v.y & 0xFFFFu) | (v.w << 16);
            o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
            xs[(p & 3) * ldsw + (p >> 2)] = o;
        }
        if (tid < 4) xs[tid * ldsw + TC] = uint4{0, 0, 0, 0};
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            if (PARTIAL && j >= jn) break;
            float d[R];
#pragma unroll
            for (int r = 0; r < R; ++r) d[r] = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 xq = xs[q * ldsw + xcol[j]];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t u = q == 0 ? wv[r][j].x : q == 1 ? wv[r][j].y
                                     : q == 2 ? wv[r][j].z : wv[r][j].w;
                    const uint32_t u8 = u >> 8;
                    const f16x2 qa = as_f16x2((u & 0x000F000Fu) ^ 0x64086408u) + bias_lo;
                    const f16x2 qb = as_f16x2((u & 0x00F000F0u) ^ 0x54805480u) + bias_hi;
                    const f16x2 qc = as_f16x2((u8 & 0x000F000Fu) ^ 0x64086408u) + bias_lo;
                    const f16x2 qd = as_f16x2((u8 & 0x00F000F0u) ^ 0x54805480u) + bias_hi;
                    d[r] = __builtin_amdgcn_fdot2(qa, as_f16x2(xq.x), d[r], false);
                    d[r] = __builtin_amdgcn_fdot2(qb, as_f16x2(xq.y), d[r], false);
                    d[r] = __builtin_amdgcn_fdot2(qc, as_f16x2(xq.z), d[r], false);
                    d[r] = __builtin_amdgcn_fdot2(qd, as_f16x2(xq.w), d[r], false);
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = __builtin_fmaf(h2f(sv[r][j]), d[r], acc[r]);
        }
        __syncthreads();
    };
    int c0 = 0;
    for (; c0 + TC <= nchunks; c0 += TC) tile.template operator()<false>(c0, TC);
    if (c0 < nchunks) tile.template operator()<true>(c0, nchunks - c0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float a = segment_sum<64>(acc[r]);
        if (col == 63 && row0 + r < n) y[row0 + r] = f2h(a);
    }
}

template <int NT, int TJ, int R>
__global__ __launch_bounds__(NT) void qgemv_tiled_kernel(
        const uint4* __restrict__ w, const float* __restrict__ scale,
        const uint4* __restrict__ x, uint16_t* __restrict__ y, int n,
        int nchunks) {
    extern __shared__ uint4 xs[];                  // [2][TC + 1]
    constexpr int TC = TJ * 64;
    constexpr int XPER = 2 * TC / NT;
    static_assert(2 * TC % NT == 0, "a tile's pieces divide over the workgroup");
    constexpr int ldsw = TC + 1;
    const int tid = threadIdx.x;
    const int col = tid & 63;
    const int64_t row0 = (static_cast<int64_t>(xcd_contiguous_block()) * (NT >> 6) + (tid >> 6)) * R;
    const char* wrow[R];
    float sc[R];   // row scales, loaded first so the final scaling waits on nothing
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint64_t rc = static_cast<uint64_t>(std::min<int64_t>(row0 + r, n - 1));
        wrow[r] = reinterpret_cast<const char*>(w) + rc * (static_cast<uint32_t>(nchunks) * 16u);
        sc[r] = scale[rc];
    }
    const f16x2 bias = {static_cast<_Float16>(-1152.0f),
                        static_cast<_Float16>(-1152.0f)};
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    auto tile = [&]<bool PARTIAL>(int c0, int tc) {
        const int jn = PARTIAL ? (tc + 63) >> 6 : TJ;
        const int np = 2 * tc;
        const uint4* xt = x + 2 * static_cast<int64_t>(c0);
        uint4 xv[XPER];
#pragma unroll
        for (int i = 0; i < XPER; ++i) xv[i] = xt[std::min(tid + i * NT, np - 1)];
        __builtin_amdgcn_sched_barrier(0);
        uint4 wv[R][TJ];
        int xcol[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            if (PARTIAL && j >= jn) break;
            const int c = col + 64 * j;
            const uint32_t cl = static_cast<uint32_t>(c0 + (c < tc ? c : tc - 1));
            xcol[j] = c < tc ? c : TC;
#pragma unroll
            for (int r = 0; r < R; ++r)
                wv[r][j] = *reinterpret_cast<const uint4*>(wrow[r] + cl * 16u);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < XPER; ++i) {
            const int p = std::min(tid + i * NT, np - 1);
            const uint4 v = xv[i];
            uint4 o;
            o.x = (v.x & 0xFFFFu) | (v.y << 16);
            o.y = (v.x >> 16) | (v.y & 0xFFFF0000u);
            o.z = (v.z & 0xFFFFu) | (v.w << 16);
            o.w = (v.z >> 16) | (v.w & 0xFFFF0000u);
            xs[(p & 1) * ldsw + (p >> 1)] = o;
        }
        if (tid < 2) xs[tid * ldsw + TC] = uint4{0, 0, 0, 0};
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            if (PARTIAL && j >= jn) break;
            const uint4 x0 = xs[xcol[j]];
            const uint4 x1 = xs[ldsw + xcol[j]];
            const uint32_t xpair[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t words[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z, wv[r][j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t u = words[q];
                    const f16x2 qp = as_f16x2((u & 0x00FF00FFu) ^ 0x64806480u) + bias;
                    const f16x2 qq = as_f16x2(((u >> 8) & 0x00FF00FFu) ^ 0x64806480u) + bias;
                    acc[r] = __builtin_amdgcn_fdot2(qp, as_f16x2(xpair[2 * q]), acc[r], false);
                    acc[r] = __builtin_amdgcn_fdot2(qq, as_f16x2(xpair[2 * q + 1]), acc[r], false);
                }
            }
        }
        __syncthreads();
    };
    int c0 = 0;
    for (; c0 + TC <= nchunks; c0 += TC) tile.template operator()<false>(c0, TC);
    if (c0 < nchunks) tile.template operator()<true>(c0, nchunks - c0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float a = segment_sum<64>(acc[r]);
        const int64_t row = row0 + r;
        if (col == 63 && row < n) y[row] = f2h(sc[r] * a);
    }
}

// Tile size of the K-tiled kernels (chunks per lane per tile); 256-thread
// workgroups throughout.  Measured on MI355X over HBM-cold pools, every
// instance bit-identical:
// - INT4, one row per wave: 7 chunks per lane per tile.  Against 8 it avoids
//   a small last tile (k = 28672 splits into two full tiles of 7): 1-13%
//   faster at 512..3072 x 20480..53248, level at 65536.
// - INT4, two rows per wave: 2 chunks per lane per tile while the row has at
//   most 16 chunks per lane (k <= 32768, at most 8 tiles): 2-8% faster than 4
//   at 4096..16384 x 20480..28672; with more tiles the barriers cost more
//   than the smaller tile saves (4096x65536: 5% slower), so 4 there.
// - INT8 (tiles of an even number of chunks, so that a tile's x pieces
//   divide over the workgroup): two rows per wave with 4 chunks per lane
//   per tile, one row with 8.  2, 6 and 14 were no faster (14 spills).
constexpr int int4_tile_j(int r, int j) { return r == 1 ? 7 : (j <= 16 ? 2 : 4); }
constexpr int q8_tile_j(int r) { return r == 2 ? 4 : 8; }
// LDS bytes of one tile of `tj` chunks per lane: `pieces` 16-byte x pieces
// per chunk (INT4 4, INT8 2), plus the zero column.
constexpr uint32_t tile_lds(int pieces, int tj) {
    return static_cast<uint32_t>(pieces) * (tj * 64 + 1) * 16u;
}

// Several independent problems of one k per launch (grouped GEMV).  The
// problem table travels by value in the kernel arguments; logical
// workgroups [start[p], start[p+1]) belong to problem p, and each computes
// exactly the rows it would compute in a launch of that problem alone, so
// the outputs are bit-identical to separate launches.
struct GroupArgs {
    const void* w[kMaxGroup];
    const void* scale[kMaxGroup];
    const void* x[kMaxGroup];
    void* y[kMaxGroup];
    int n[kMaxGroup];
    uint32_t start[kMaxGroup + 1];
    int count;
};

__device__ __forceinline__ int group_of(const GroupArgs& g, uint32_t lb) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i) p += (i < g.count && lb >= g.start[i]) ? 1 : 0;
    return p;
}

template <int CW, int J, int R, int NT>
__global__ __launch_bounds__(NT) void int4gemv_lds_group_kernel(GroupArgs g,
                                                                 int nchunks) {
    extern __shared__ uint4 xs[];
    const uint32_t lb = xcd_contiguous_block();
    const int p = group_of(g, lb);
    int4_lds_rows<CW, J, R, NT>(static_cast<const uint4*>(g.w[p]),
                                static_cast<const uint16_t*>(g.scale[p]),
                                static_cast<const uint4*>(g.x[p]),
                                static_cast<uint16_t*>(g.y[p]), g.n[p], nchunks,
                                lb - g.start[p], xs);
}

template <int CW, int J, int R, int NT>
__global__ __launch_bounds__(NT) void qgemv_lds_group_kernel(GroupArgs g,
                                                             int nchunks) {
    extern __shared__ uint4 xs[];
    const uint32_t lb = xcd_contiguous_block();
    const int p = group_of(g, lb);
    q8_lds_rows<CW, J, R, NT>(static_cast<const uint4*>(g.w[p]),
                              static_cast<const float*>(g.scale[p]),
                              static_cast<const uint4*>(g.x[p]),
                              static_cast<uint16_t*>(g.y[p]), g.n[p], nchunks,
                              lb - g.start[p], xs);
}


// ------------------------------------------------------------- FP16/FP32
//
// The reference's FP16/FP32 GEMV (kernels/gemv/gemv_common.h:1-79):
// y[n] = sum_k W[n,k] * x[k] accumulated in FP32 and cast once to the
// dtype of W (RNE for fp16).  W and x are fp16 or fp32, same dtype.

__device__ __forceinline__ float fp_to_f(uint16_t h) { return h2f(h); }
__device__ __forceinline__ float fp_to_f(float f) { return f; }
__device__ __forceinline__ void fp_store(uint16_t* p, float v) { *p = f2h(v); }
__device__ __forceinline__ void fp_store(float* p, float v) { *p = v; }

// One 16-byte chunk of W against the matching chunk of x, into acc, one
// FMA per element: fp16 operands go straight into v_fma_mix_f32 (the
// fp16 x fp16 product is exact in FP32, the add is one round-to-nearest-
// even), fp32 as plain FMAs.  v_dot2_f32_f16 would halve the instructions
// but measured on gfx950 it is not a single RNE rounding (about 1% of
// random operands differ from one, in a sign-asymmetric way), and this
// path is memory-bound at 2 or 4 bytes per element, so the FMA costs
// nothing.
__device__ __forceinline__ float fma_pair(uint32_t w, uint32_t x, float acc) {
    const f16x2 a = as_f16x2(w), b = as_f16x2(x);
    acc = __builtin_fmaf(static_cast<float>(a[0]), static_cast<float>(b[0]), acc);
    return __builtin_fmaf(static_cast<float>(a[1]), static_cast<float>(b[1]), acc);
}
// Four independent accumulators per lane (one per 32-bit word of a chunk)
// keep consecutive FMAs free of dependencies; they are summed at the end.
__device__ __forceinline__ void dot_chunk(uint16_t, const uint4& w,
                                          const uint4& x, float (&acc)[4]) {
    acc[0] = fma_pair(w.x, x.x, acc[0]);
    acc[1] = fma_pair(w.y, x.y, acc[1]);
    acc[2] = fma_pair(w.z, x.z, acc[2]);
    acc[3] = fma_pair(w.w, x.w, acc[3]);
}
__device__ __forceinline__ void dot_chunk(float, const uint4& w,
                                          const uint4& x, float (&acc)[4]) {
    acc[0] = __builtin_fmaf(__builtin_bit_cast(float, w.x), __builtin_bit_cast(float, x.x), acc[0]);
    acc[1] = __builtin_fmaf(__builtin_bit_cast(float, w.y), __builtin_bit_cast(float, x.y), acc[1]);
    acc[2] = __builtin_fmaf(__builtin_bit_cast(float, w.z), __builtin_bit_cast(float, x.z), acc[2]);
    acc[3] = __builtin_fmaf(__builtin_bit_cast(float, w.w), __builtin_bit_cast(float, x.w), acc[3]);
}

// Scalar: one 256-thread workgroup per row, element loads.  The single
// source of gemv_baseline and of every fallback (bit-identity of the two).
template <typename S>
__global__ __launch_bounds__(kBlock) void gemv_scalar_kernel(
        const S* __restrict__ w, const S* __restrict__ x, S* __restrict__ y,
        int64_t k) {
    const int64_t row = blockIdx.x;
    const S* __restrict__ wrow = w + row * k;
    float acc = 0.f;
    for (int64_t i = threadIdx.x; i < k; i += kBlock)
        acc = __builtin_fmaf(fp_to_f(wrow[i]), fp_to_f(x[i]), acc);
    acc = segment_sum<64>(acc);
    __shared__ float part[kBlock / 64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 63) part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) fp_store(y + row, (part[0] + part[1]) + (part[2] + part[3]));
}

// Vector: CW lanes per row (64/CW rows per wave), lane `col` owns the
// 16-byte chunks col + CW*j.  x is staged once per workgroup in LDS
// ([nchunks + 1] chunks, the last one zero: what lanes past the row end
// read).  The lane's W chunks stream through two register batches of JB
// chunks: batch b+1 is in flight while batch b is multiplied, so any K
// runs with a bounded register budget.
constexpr int kGemvBatch = 8;

// JB: chunks per lane per register batch, the smaller of kGemvBatch and
// the lane's chunk count rounded up to a power of two (a batch longer than
// the row would load and multiply padding).
template <typename S, int CW, int NT, int JB>
__global__ __launch_bounds__(NT) void gemv_lds_kernel(
        const uint4* __restrict__ w,   // [n][nchunks] 16-byte chunks
        const uint4* __restrict__ x,   // [nchunks] 16-byte chunks
        S* __restrict__ y, int n, int nchunks) {
    extern __shared__ uint4 xs[];
    constexpr int SLOTS = 64 / CW;
    constexpr int XB = 4;              // x chunks per thread per staging pass
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int col = lane % CW;
    const int slot = lane / CW;
    const uint32_t blk = xcd_contiguous_block();
    const int64_t row =
        (static_cast<int64_t>(blk) * (NT >> 6) + (tid >> 6)) * SLOTS + slot;
    const uint32_t rowc = static_cast<uint32_t>(std::min<int64_t>(row, n - 1));
    const char* wb = reinterpret_cast<const char*>(w);
    const uint32_t wrow_bytes = static_cast<uint32_t>(nchunks) * 16u;
    const int nbatch = ((nchunks + CW - 1) / CW + JB - 1) / JB;

    // x first (the barrier waits for it), in passes of XB chunks per thread
    uint4 xv[XB];
#pragma unroll
    for (int i = 0; i < XB; ++i) xv[i] = x[std::min(tid + i * NT, nchunks - 1)];
    __builtin_amdgcn_sched_barrier(0);
    uint4 wa[JB], wn[JB];
    auto load = [&](uint4 (&dst)[JB], int b) {
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            const int c = col + CW * (b * JB + jj);
            const uint32_t cl = static_cast<uint32_t>(c < nchunks ? c : nchunks - 1);
            dst[jj] = *reinterpret_cast<const uint4*>(wb + (rowc * wrow_bytes + cl * 16u));
        }
    };
    load(wa, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < XB; ++i) xs[std::min(tid + i * NT, nchunks - 1)] = xv[i];
    for (int base = XB * NT; base < nchunks; base += XB * NT) {   // K beyond one pass
#pragma unroll
        for (int i = 0; i < XB; ++i) {
            const int c = std::min(base + tid + i * NT, nchunks - 1);
            xs[c] = x[c];
        }
    }
    if (tid == 0) xs[nchunks] = uint4{0, 0, 0, 0};
    __syncthreads();

    float accs[4] = {0.f, 0.f, 0.f, 0.f};
    auto comp = [&](const uint4 (&src)[JB], int b) {
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            const int c = col + CW * (b * JB + jj);
            dot_chunk(S{}, src[jj], xs[c < nchunks ? c : nchunks], accs);
        }
    };
    for (int b = 0; b < nbatch; b += 2) {
        if (b + 1 < nbatch) load(wn, b + 1);
        comp(wa, b);
        if (b + 1 < nbatch) {
            if (b + 2 < nbatch) load(wa, b + 2);
            comp(wn, b + 1);
        }
    }
    float acc = (accs[0] + accs[1]) + (accs[2] + accs[3]);
    acc = segment_sum<CW>(acc);
    if (col == CW - 1 && row < n) fp_store(y + row, acc);
}

// K-tiled FP16/FP32 GEMV, for rows whose x does not fit the 64 KiB stage
// (k > 32768 fp16, > 16384 fp32; gemv_lds_tiled forces it at any k).  64
// lanes per row, one row per wave.  x is staged tile by tile (kGemvTileJ
// chunks per lane per tile, 32 KB), with a barrier before the tile is read
// and one before the next tile overwrites it; every thread runs the same
// tiles (they depend on nchunks only; rows past n are clamped), so every
// barrier is reached by all.  Within a tile the lane's W chunks stream
// through two register batches of kGemvBatch chunks as in gemv_lds_kernel.
// Lane `col` takes chunks col + 64 j in j order, so where x fits one stage
// the sums are bit-identical to gemv_lds_kernel with CW = 64.
constexpr int kGemvTileJ = 4 * kGemvBatch;    // 32 chunks per lane per tile
constexpr uint32_t kGemvTileLds = (kGemvTileJ * 64 + 1) * 16u;   // 32,784 B

template <typename S, int NT>
__global__ __launch_bounds__(NT) void gemv_tiled_kernel(
        const uint4* __restrict__ w,   // [n][nchunks] 16-byte chunks
        const uint4* __restrict__ x,   // [nchunks] 16-byte chunks
        S* __restrict__ y, int n, int nchunks) {
    extern __shared__ uint4 xs[];                 // [TC + 1], the last zero
    constexpr int JB = kGemvBatch;
    constexpr int TC = kGemvTileJ * 64;           // chunks per tile
    constexpr int XPER = TC / NT;                 // x chunks per thread per tile
    static_assert(TC % NT == 0, "a tile's chunks divide over the workgroup");
    const int tid = threadIdx.x;
    const int col = tid & 63;
    const int64_t row = static_cast<int64_t>(xcd_contiguous_block()) * (NT >> 6) + (tid >> 6);
    const uint64_t rowc = static_cast<uint64_t>(std::min<int64_t>(row, n - 1));
    const char* wrow = reinterpret_cast<const char*>(w) +
                       rowc * (static_cast<uint32_t>(nchunks) * 16u);
    float accs[4] = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nchunks; c0 += TC) {
        const int tc = std::min(TC, nchunks - c0);            // chunks in this tile
        const int nbatch = ((tc + 63) / 64 + JB - 1) / JB;    // wave-uniform
        const uint4* xt = x + c0;
        uint4 xv[XPER];
#pragma unroll
        for (int i = 0; i < XPER; ++i) xv[i] = xt[std::min(tid + i * NT, tc - 1)];
        __builtin_amdgcn_sched_barrier(0);
        uint4 wa[JB], wn[JB];
        auto load = [&](uint4 (&dst)[JB], int b) {
#pragma unroll
            for (int jj = 0; jj < JB; ++jj) {
                const int c = col + 64 * (b * JB + jj);
                const uint32_t cl = static_cast<uint32_t>(c0 + (c < tc ? c : tc - 1));
                dst[jj] = *reinterpret_cast<const uint4*>(wrow + cl * 16u);
            }
        };
        load(wa, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < XPER; ++i) xs[std::min(tid + i * NT, tc - 1)] = xv[i];
        if (tid == 0) xs[TC] = uint4{0, 0, 0, 0};
        __syncthreads();
        auto comp = [&](const uint4 (&src)[JB], int b) {
#pragma unroll
            for (int jj = 0; jj < JB; ++jj) {
                const int c = col + 64 * (b * JB + jj);
                dot_chunk(S{}, src[jj], xs[c < tc ? c : TC], accs);
            }
        };
        for (int b = 0; b < nbatch; b += 2) {
            if (b + 1 < nbatch) load(wn, b + 1);
            comp(wa, b);
            if (b + 1 < nbatch) {
                if (b + 2 < nbatch) load(wa, b + 2);
                comp(wn, b + 1);
            }
        }
        __syncthreads();
    }
    float acc = (accs[0] + accs[1]) + (accs[2] + accs[3]);
    acc = segment_sum<64>(acc);
    if (col == 63 && row < n) fp_store(y + row, acc);
}

// ------------------------------------------------- read-only ceiling
//
// A plain streaming read of `bytes`, one 16-byte load per thread.  Of the
// read patterns measured for one 8.67 MB launch over an HBM-cold pool (1, 2,
// 4, 8 or 16 loads per thread at 256, 512 or 1024 threads, strided or
// contiguous, with and without the nontemporal hint), one load per thread
// in 256-thread workgroups was fastest (2.89 us; 4 loads per thread 3.18 us,
// 16 loads 3.49 us): the most waves, each with the shortest dependency.  The
// loaded words are folded and compared with `key`, a launch argument the
// compiler cannot see, so the loads cannot be removed; the store to `sink`
// runs only if a thread's fold equals the key (harmless either way: sink is
// the caller's scratch word).  It is the measured bandwidth ceiling of one
// launch that reads the same number of bytes as a GEMV call.
__global__ __launch_bounds__(kBlock) void stream_read_kernel(
        const uint4* __restrict__ p, uint32_t* __restrict__ sink, int64_t n16,
        uint32_t key) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const uint4 v = p[idx < n16 ? idx : n16 - 1];
    const uint32_t a = v.x ^ v.y ^ v.z ^ v.w;
    if (a == key) sink[0] = a;
}

// A workgroup that does no memory work: launched back to back on one stream
// it measures what one dispatch of a given grid and workgroup size costs
// before any kernel body runs (command processing, workgroup launch, the
// end-of-kernel release).  The store is never taken: the host passes a key
// no thread index reaches.
__global__ __launch_bounds__(1024) void empty_launch_kernel(
        uint32_t* __restrict__ sink, uint32_t key) {
    if (threadIdx.x == key) sink[0] = blockIdx.x;
}

// A bounded on-device wait for the timing loops: one wave sleeps until the
// constant-rate wall clock has advanced `ticks`, or until it has gone round
// its loop `max_iters` times, whichever comes first (so it ends even if the
// clock were not running).  Queued ahead of a timed window it keeps the GPU
// busy while the host enqueues the window's launches, so the window times
// the GPU and not the host's submission rate (about 2.5-3.5 us per launch
// on MI355X, close to a short GEMV's own time).  It touches no memory.
__global__ __launch_bounds__(64) void delay_kernel(uint64_t ticks,
                                                   uint64_t max_iters) {
    const uint64_t t0 = wall_clock64();
    for (uint64_t i = 0; i < max_iters; ++i) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(8);
    }
}

// --------------------------------------------------------- instance tables

using Int4Fn = void (*)(const uint4*, const uint16_t*, const uint4*,
                        uint16_t*, int, int);
using Q8Fn = void (*)(const uint4*, const float*, const uint4*, uint16_t*,
                      int, int);

// One traits type per kernel family: the instance for (CW, J, R), or null
// where the register budget does not allow R rows per lane at J chunks.
struct Int4Wave {
    using Fn = Int4Fn;
    static constexpr int kMaxJ = kInt4MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (R <= int4_rmax(J)) return &int4gemv_wave_kernel<CW, J, R>;
        else return nullptr;
    }
};
// The INT4 plans take 512-thread workgroups only with one row per lane
// (lds_threads), so only those instances exist at 512 threads.
template <int NT, int R>
constexpr bool int4_lds_shape(int j) {
    return R <= int4_rmax(j) && (NT != 512 || R == 1);
}
template <int NT>
struct Int4Lds {
    using Fn = Int4Fn;
    static constexpr int kMaxJ = kInt4MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (int4_lds_shape<NT, R>(J)) return &int4gemv_lds_kernel<CW, J, R, NT>;
        else return nullptr;
    }
};
struct Q8Wave {
    using Fn = Q8Fn;
    static constexpr int kMaxJ = kQ8MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (R <= q8_rmax(J)) return &qgemv_wave_kernel<CW, J, R>;
        else return nullptr;
    }
};
template <int NT>
struct Q8Lds {
    using Fn = Q8Fn;
    static constexpr int kMaxJ = kQ8MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (R <= q8_rmax(J)) return &qgemv_lds_kernel<CW, J, R, NT>;
        else return nullptr;
    }
};

using Int4StampFn = void (*)(const uint4*, const uint16_t*, const uint4*,
                             uint16_t*, int, int, uint64_t*);
template <int NT>
struct Int4LdsStamp {
    using Fn = Int4StampFn;
    static constexpr int kMaxJ = kInt4MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (int4_lds_shape<NT, R>(J)) return &int4gemv_lds_stamp_kernel<CW, J, R, NT>;
        else return nullptr;
    }
};

using Int4GroupFn = void (*)(GroupArgs, int);
using Q8GroupFn = void (*)(GroupArgs, int);

template <int NT>
struct Int4LdsGroup {
    using Fn = Int4GroupFn;
    static constexpr int kMaxJ = kInt4MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (R <= int4_rmax(J)) return &int4gemv_lds_group_kernel<CW, J, R, NT>;
        else return nullptr;
    }
};
template <int NT>
struct Q8LdsGroup {
    using Fn = Q8GroupFn;
    static constexpr int kMaxJ = kQ8MaxJ;
    template <int CW, int J, int R>
    static constexpr Fn get() {
        if constexpr (R <= q8_rmax(J)) return &qgemv_lds_group_kernel<CW, J, R, NT>;
        else return nullptr;
    }
};

constexpr int r_index(int r) { return r == 1 ? 0 : (r == 2 ? 1 : 2); }

template <class F, int CW, int J>
typename F::Fn pick_r(int r) {
    static constexpr typename F::Fn t[3] = {F::template get<CW, J, 1>(),
                                            F::template get<CW, J, 2>(),
                                            F::template get<CW, J, 4>()};
    return t[r_index(r)];
}

template <class F, int... Js>
typename F::Fn pick_j64(int j, int r, std::integer_sequence<int, Js...>) {
    typename F::Fn f = nullptr;
    ((j == Js + 1 ? (f = pick_r<F, 64, Js + 1>(r), 0) : 0), ...);
    return f;
}

template <class F>
typename F::Fn instance(int cw, int j, int r) {
    if (cw == 16 && j == 1) return pick_r<F, 16, 1>(r);
    if (cw == 32 && j == 1) return pick_r<F, 32, 1>(r);
    if (cw == 64 && j >= 1 && j <= F::kMaxJ)
        return pick_j64<F>(j, r, std::make_integer_sequence<int, F::kMaxJ>{});
    return nullptr;
}

// Launch with the argument types taken from the kernel's own signature.
template <typename... Params>
hipError_t launch(void (*kernel)(Params...), int64_t grid, int block,
                  uint32_t shmem, hipStream_t stream, hipEvent_t ev0,
                  hipEvent_t ev1, std::type_identity_t<Params>... args) {
    void* argv[] = {static_cast<void*>(&args)...};
    const dim3 g(static_cast<uint32_t>(grid)), b(static_cast<uint32_t>(block));
    if (ev0 == nullptr && ev1 == nullptr)
        return hipLaunchKernel(reinterpret_cast<const void*>(kernel), g, b,
                               argv, shmem, stream);
    return hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), g, b,
                              argv, shmem, stream, ev0, ev1, 0);
}

// The same launch resolved into a Launch record instead of enqueued: the
// kernel, its shape and its arguments, each argument copied into an 8-byte
// slot (the runtime reads each argument's own size from the slot's start).
template <typename... Params>
hipError_t bind(Launch* out, void (*kernel)(Params...), int64_t grid,
                int block, uint32_t shmem, std::type_identity_t<Params>... args) {
    static_assert(sizeof...(Params) <= kMaxLaunchArgs, "too many kernel arguments");
    static_assert(((sizeof(Params) <= 8 && std::is_trivially_copyable_v<Params>) && ...),
                  "kernel arguments must fit an 8-byte slot");
    if (grid < 1 || grid > UINT32_MAX) return hipErrorInvalidConfiguration;
    Launch L;
    L.fn = reinterpret_cast<const void*>(kernel);
    L.grid = static_cast<uint32_t>(grid);
    L.block = static_cast<uint32_t>(block);
    L.shmem = shmem;
    L.nargs = sizeof...(Params);
    int i = 0;
    ((std::memcpy(&L.args[i++], &args, sizeof(args))), ...);
    *out = L;
    return hipSuccess;
}

int pow2_at_least(int64_t v, int lo) {
    int p = lo;
    while (p < v && p < 64) p <<= 1;
    return p;
}

// Default rows per lane (measured on MI355X with kernel arguments
// preloaded, HBM-cold pools, back-to-back launches on a pre-filled queue;
// every candidate bit-identical).  INT4 with at most 3 chunks per lane:
// - rows of at most 32 chunks (64 // CW >= 2 row slots per wave): two rows
//   (4096x1024: 2.39 us against 2.55);
// - otherwise one row while one row per wave keeps the whole grid resident
//   (at most 32 waves per CU on kCus CUs), two above, where one row per wave
//   would run a second round of waves: 4096^2 one row 3.38 us against two
//   3.56-3.63; 6144x4096 4.18 against 4.34; 11008x4096 two rows 6.05 against
//   6.36; 14336x4096 7.41 against 7.65; 13824x5120 9.32 against 10.14.
// With 4 or more chunks per lane one row throughout (8192^2 8.19 us against
// 9.01, 28672x8192 24.3 against 25.0).  INT8 does best with one row per lane
// at every shape measured.
constexpr int64_t kCus = 256;
constexpr int64_t kResidentWaves = 32 * kCus;
int default_rows_int4(int64_t n, int slots, int j, int rmax) {
    if (j > 3 || rmax < 2) return 1;
    if (slots >= 2) return 2;
    return n > kResidentWaves ? 2 : 1;
}

// Workgroup size of the LDS kernels.  512 threads halve the number of
// workgroups that stage x.  Measured on MI355X (same launch path, HBM-cold
// pools) this pays when x is large next to each workgroup's weights (INT4
// with one row per lane, INT8 with 8+ chunks per lane: 4096x11008 INT4
// 7.44 -> 6.93 us, INT8 10.48 -> 9.88 us) and the 512-thread grid fills the
// CUs in whole rounds (a multiple of kCus workgroups) or runs many (8+) of
// them.  A partial round among few costs
// more than the staging saves: 5120x13824 (640 workgroups of 512, 2.5
// rounds; 1280 of 256) INT4 10.2 us with 512 threads, 9.8 with 256, INT8
// 15.4 and 14.6; 5120^2 INT4 5.15 and 4.8.  Among many rounds the partial
// one matters less: 27648x5120 (13.5 rounds) 15.8-16.0 us with 512, 16.0-16.3
// with 256.  INT8 at K = 4096 was 1-3% slower with 512.
// True when `waves` in 512-thread workgroups fill the CUs in whole rounds
// or in 8+ rounds (the condition for 512-thread plans, all operators).
bool rounds_ok_512(int64_t waves) {
    const int64_t grid = (waves + 7) / 8;
    return grid >= kCus && (grid % kCus == 0 || grid >= 8 * kCus);
}

int lds_threads(bool int4, int r, int j, int64_t waves) {
    const bool rounds_ok = rounds_ok_512(waves);
    // INT4: 512 threads with one row per lane (4096^2 3.38 us against 3.43,
    // 4096x11008 6.82 against 7.14, 8192^2 8.19 against 8.48); with two
    // rows 256 threads (11008x4096 6.05 against 6.14, 13824x5120 9.32
    // against 10.30)
    if (int4 && r == 1 && rounds_ok) return 512;
    if (!int4 && j >= 8 && rounds_ok) return 512;
    return kBlock;
}

void finish_wave_plan(Plan& p, int64_t n, bool int4) {
    const int slots = 64 / p.cw;
    const int64_t rows_per_wave = static_cast<int64_t>(slots) * p.r;
    const int64_t waves = (n + rows_per_wave - 1) / rows_per_wave;
    // the LDS kernels stage x with every thread of a full block
    const int64_t block_waves =
        p.kind == kLds ? lds_threads(int4, p.r, p.j, waves) / 64
                       : std::min<int64_t>(kBlock / 64, waves);
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

// The K-tiled kernel: `rows` rows per wave if requested (1 or 2), else one
// up to n = 3072 and two above.  Up to 3072 rows one row per wave (n / 4
// workgroups, at most 3 per CU) with the longer tile keeps more bytes in
// flight: INT4 2048 and 3072 x 28672 10-11% faster than two rows, INT8
// 2048x28672 15%, 2048x65536 13%, 3072x28672 level.  From 3328 rows two rows
// per wave are faster for both (INT4 3328x28672 7%, INT8 3328x28672 11%,
// 3584x65536 6%): one row would leave a fourth, partial workgroup on some CUs.
Plan tiled_plan(int rows, int64_t n, int64_t nchunks, bool int4) {
    Plan p;
    p.kind = kTiled;
    p.cw = 64;
    p.j = static_cast<int>((nchunks + 63) / 64);
    p.r = rows > 0 ? std::min(rows, 2) : (n > 3072 ? 2 : 1);
    p.tile = int4 ? int4_tile_j(p.r, p.j) : q8_tile_j(p.r);
    p.block = kBlock;
    const int64_t waves = (n + p.r - 1) / p.r;
    p.grid = (waves + kBlock / 64 - 1) / (kBlock / 64);
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
    const int64_t nchunks = k / 32;
    // the untiled LDS kernels address W with 32-bit byte offsets; the tiled
    // kernel keeps 64-bit row bases, so it also takes weights of 4 GiB or more
    const bool big = n * (k / 2) >= (int64_t{1} << 32);
    if (kind == kTiled || (kind == kLds && (k > kMaxWaveK || big)))
        return tiled_plan(rows, n, nchunks, true);
    if (k > kMaxWaveK) return scalar_plan(n, true, "k above the wave kernels' register-resident x");
    Plan p;
    p.kind = kind;
    p.cw = pow2_at_least(nchunks, 16);
    p.j = static_cast<int>((nchunks + p.cw - 1) / p.cw);
    const int rmax = int4_rmax(p.j);
    p.r = rows > 0 ? std::min(rows, rmax) : default_rows_int4(n, 64 / p.cw, p.j, rmax);
    if (p.r == 3) p.r = 2;
    finish_wave_plan(p, n, true);
    return p;
}

Plan plan_q8(int kind, int rows, int64_t n, int64_t k, const void* w,
             const void* x) {
    if (kind == kScalar) return scalar_plan(n, false, "");
    if (!q8_contract_ok(w, x, k))
        return scalar_plan(n, true, "vector contract unmet (w/x 16B alignment, k%16)");
    const int64_t nchunks = k / 16;
    const bool big = n * k >= (int64_t{1} << 32);    // as in plan_int4
    if (kind == kTiled || (kind == kLds && (k > kMaxWaveK || big)))
        return tiled_plan(rows, n, nchunks, false);
    if (k > kMaxWaveK) return scalar_plan(n, true, "k above the wave kernels' register-resident x");
    Plan p;
    p.kind = kind;
    p.cw = pow2_at_least(nchunks, 16);
    p.j = static_cast<int>((nchunks + p.cw - 1) / p.cw);
    const int rmax = q8_rmax(p.j);
    p.r = rows > 0 ? std::min(rows, rmax) : 1;
    if (p.r == 3) p.r = 2;
    finish_wave_plan(p, n, false);
    return p;
}

hipError_t prepare_int4(const Plan& p, const void* w, const void* scale,
                        const void* x, void* y, int64_t n, int64_t k, Launch* L) {
    if (p.kind == kScalar)
        return bind(L, int4gemv_scalar_kernel, p.grid, p.block, 0,
                    static_cast<const uint8_t*>(w),
                    static_cast<const uint16_t*>(scale),
                    static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), k);
    if (p.kind == kTiled) {
        const Int4Fn tfn =
            p.r == 1 && p.tile == 7   ? &int4gemv_tiled_kernel<kBlock, 7, 1>
            : p.r == 2 && p.tile == 2 ? &int4gemv_tiled_kernel<kBlock, 2, 2>
            : p.r == 2 && p.tile == 4 ? &int4gemv_tiled_kernel<kBlock, 4, 2>
                                      : nullptr;
        if (tfn == nullptr) return hipErrorInvalidConfiguration;
        return bind(L, tfn, p.grid, kBlock, tile_lds(4, p.tile),
                    static_cast<const uint4*>(w), static_cast<const uint16_t*>(scale),
                    static_cast<const uint4*>(x), static_cast<uint16_t*>(y),
                    static_cast<int>(n), static_cast<int>(k / 32));
    }
    const Int4Fn fn =
        p.kind == kWave ? instance<Int4Wave>(p.cw, p.j, p.r)
        : p.block == 512 ? instance<Int4Lds<512>>(p.cw, p.j, p.r)
                         : instance<Int4Lds<kBlock>>(p.cw, p.j, p.r);
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    if (p.kind == kLds && !lds_chunks_ok(p, k / 32)) return hipErrorInvalidConfiguration;
    const uint32_t shmem = p.kind == kLds ? int4_lds_bytes(p.cw, p.j) : 0;
    return bind(L, fn, p.grid, p.block, shmem, static_cast<const uint4*>(w),
                static_cast<const uint16_t*>(scale), static_cast<const uint4*>(x),
                static_cast<uint16_t*>(y), static_cast<int>(n),
                static_cast<int>(k / 32));
}

hipError_t prepare_q8(const Plan& p, const void* w, const void* scale,
                      const void* x, void* y, int64_t n, int64_t k, Launch* L) {
    if (p.kind == kScalar)
        return bind(L, qgemv_scalar_kernel, p.grid, p.block, 0,
                    static_cast<const int8_t*>(w), static_cast<const float*>(scale),
                    static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), k);
    if (p.kind == kTiled) {
        const Q8Fn tfn = p.r == 2 && p.tile == q8_tile_j(2) ? &qgemv_tiled_kernel<kBlock, q8_tile_j(2), 2>
                         : p.r == 1 && p.tile == q8_tile_j(1) ? &qgemv_tiled_kernel<kBlock, q8_tile_j(1), 1>
                                                               : nullptr;
        if (tfn == nullptr) return hipErrorInvalidConfiguration;
        return bind(L, tfn, p.grid, kBlock, tile_lds(2, p.tile),
                    static_cast<const uint4*>(w), static_cast<const float*>(scale),
                    static_cast<const uint4*>(x), static_cast<uint16_t*>(y),
                    static_cast<int>(n), static_cast<int>(k / 16));
    }
    const Q8Fn fn = p.kind == kWave ? instance<Q8Wave>(p.cw, p.j, p.r)
                    : p.block == 512 ? instance<Q8Lds<512>>(p.cw, p.j, p.r)
                                     : instance<Q8Lds<kBlock>>(p.cw, p.j, p.r);
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    if (p.kind == kLds && !lds_chunks_ok(p, k / 16)) return hipErrorInvalidConfiguration;
    const uint32_t shmem = p.kind == kLds ? q8_lds_bytes(p.cw, p.j) : 0;
    return bind(L, fn, p.grid, p.block, shmem, static_cast<const uint4*>(w),
                static_cast<const float*>(scale), static_cast<const uint4*>(x),
                static_cast<uint16_t*>(y), static_cast<int>(n),
                static_cast<int>(k / 16));
}

hipError_t enqueue(const Launch& L, hipStream_t stream, hipEvent_t ev0,
                   hipEvent_t ev1) {
    if (L.fn == nullptr || L.nargs > kMaxLaunchArgs) return hipErrorInvalidConfiguration;
    void* argv[kMaxLaunchArgs];
    for (uint32_t i = 0; i < L.nargs; ++i)
        argv[i] = const_cast<uint64_t*>(&L.args[i]);
    const dim3 g(L.grid), b(L.block);
    if (ev0 == nullptr && ev1 == nullptr)
        return hipLaunchKernel(L.fn, g, b, argv, L.shmem, stream);
    return hipExtLaunchKernel(L.fn, g, b, argv, L.shmem, stream, ev0, ev1, 0);
}

hipError_t launch_int4(const Plan& p, const void* w, const void* scale,
                       const void* x, void* y, int64_t n, int64_t k,
                       hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    Launch L;
    const hipError_t e = prepare_int4(p, w, scale, x, y, n, k, &L);
    return e != hipSuccess ? e : enqueue(L, stream, ev0, ev1);
}

hipError_t launch_int4_stamped(const Plan& p, const void* w, const void* scale,
                               const void* x, void* y, int64_t n, int64_t k,
                               uint64_t* stamps, hipStream_t stream) {
    if (p.kind != kLds || !lds_chunks_ok(p, k / 32)) return hipErrorInvalidConfiguration;
    if (p.block != 512 && p.block != kBlock) return hipErrorInvalidConfiguration;
    const Int4StampFn fn = p.block == 512 ? instance<Int4LdsStamp<512>>(p.cw, p.j, p.r)
                                          : instance<Int4LdsStamp<kBlock>>(p.cw, p.j, p.r);
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    return launch(fn, p.grid, p.block, int4_lds_bytes(p.cw, p.j), stream, nullptr,
                  nullptr, static_cast<const uint4*>(w),
                  static_cast<const uint16_t*>(scale), static_cast<const uint4*>(x),
                  static_cast<uint16_t*>(y), static_cast<int>(n),
                  static_cast<int>(k / 32), stamps);
}

hipError_t launch_q8(const Plan& p, const void* w, const void* scale,
                     const void* x, void* y, int64_t n, int64_t k,
                     hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    Launch L;
    const hipError_t e = prepare_q8(p, w, scale, x, y, n, k, &L);
    return e != hipSuccess ? e : enqueue(L, stream, ev0, ev1);
}

namespace {

// Shared part of the grouped plans: the plan of the whole group's rows for
// the LDS kernel (cw, j from k; r and block from the total row count), or a
// "launch one by one" plan when any problem cannot take the LDS kernel.
template <typename PlanFn, typename OkFn>
Plan group_plan(PlanFn plan_one, OkFn lds_ok, int rows,
                const GroupProblem* probs, int count, int64_t k) {
    Plan p;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        if (!lds_ok(probs[i])) {
            p.fallback = true;
            p.why = "a problem misses the vector contract or the LDS limits";
            return p;
        }
        total += probs[i].n;
    }
    p = plan_one(kLds, rows, total, k, probs[0].w, probs[0].x);
    if (p.kind != kLds) {
        p.kind = kScalar;
        p.fallback = true;
    }
    return p;
}

// Per-problem workgroup counts of plan `p` and their prefix sums.
bool fill_group(const Plan& p, const GroupProblem* probs, int count,
                GroupArgs& g, int64_t& grid) {
    const int64_t rows_per_wave = static_cast<int64_t>(64 / p.cw) * p.r;
    const int64_t block_waves = p.block / 64;
    int64_t start = 0;
    for (int i = 0; i < kMaxGroup; ++i) {
        g.w[i] = g.scale[i] = g.x[i] = nullptr;
        g.y[i] = nullptr;
        g.n[i] = 0;
    }
    for (int i = 0; i < count; ++i) {
        const int64_t waves = (probs[i].n + rows_per_wave - 1) / rows_per_wave;
        g.w[i] = probs[i].w;
        g.scale[i] = probs[i].scale;
        g.x[i] = probs[i].x;
        g.y[i] = probs[i].y;
        g.n[i] = static_cast<int>(probs[i].n);
        g.start[i] = static_cast<uint32_t>(start);
        start += (waves + block_waves - 1) / block_waves;
        if (start > INT32_MAX) return false;
    }
    for (int i = count; i <= kMaxGroup; ++i) g.start[i] = static_cast<uint32_t>(start);
    g.count = count;
    grid = start;
    return true;
}

template <typename Fn>
hipError_t launch_group(Fn fn, const Plan& p, const GroupArgs& g,
                        int64_t grid, uint32_t shmem, int nchunks,
                        hipStream_t stream) {
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    GroupArgs a = g;
    int nc = nchunks;
    void* argv[] = {static_cast<void*>(&a), static_cast<void*>(&nc)};
    return hipLaunchKernel(reinterpret_cast<const void*>(fn),
                           dim3(static_cast<uint32_t>(grid)),
                           dim3(static_cast<uint32_t>(p.block)), argv, shmem,
                           stream);
}

}  // namespace

Plan plan_int4_group(int rows, const GroupProblem* probs, int count, int64_t k) {
    return group_plan(
        plan_int4,
        [k](const GroupProblem& q) {
            return int4_contract_ok(q.w, q.x, k) && k <= kMaxWaveK &&
                   q.n * (k / 2) < (int64_t{1} << 32);
        },
        rows, probs, count, k);
}

Plan plan_q8_group(int rows, const GroupProblem* probs, int count, int64_t k) {
    return group_plan(
        plan_q8,
        [k](const GroupProblem& q) {
            return q8_contract_ok(q.w, q.x, k) && k <= kMaxWaveK &&
                   q.n * k < (int64_t{1} << 32);
        },
        rows, probs, count, k);
}

hipError_t launch_int4_group(const Plan& p, const GroupProblem* probs,
                             int count, int64_t k, hipStream_t stream) {
    if (p.kind != kLds || count < 1 || count > kMaxGroup)
        return hipErrorInvalidConfiguration;
    GroupArgs g;
    int64_t grid = 0;
    if (!fill_group(p, probs, count, g, grid)) return hipErrorInvalidConfiguration;
    const Int4GroupFn fn = p.block == 512
                               ? instance<Int4LdsGroup<512>>(p.cw, p.j, p.r)
                               : instance<Int4LdsGroup<kBlock>>(p.cw, p.j, p.r);
    if (!lds_chunks_ok(p, k / 32)) return hipErrorInvalidConfiguration;
    return launch_group(fn, p, g, grid, int4_lds_bytes(p.cw, p.j),
                        static_cast<int>(k / 32), stream);
}

hipError_t launch_q8_group(const Plan& p, const GroupProblem* probs,
                           int count, int64_t k, hipStream_t stream) {
    if (p.kind != kLds || count < 1 || count > kMaxGroup)
        return hipErrorInvalidConfiguration;
    GroupArgs g;
    int64_t grid = 0;
    if (!fill_group(p, probs, count, g, grid)) return hipErrorInvalidConfiguration;
    const Q8GroupFn fn = p.block == 512
                             ? instance<Q8LdsGroup<512>>(p.cw, p.j, p.r)
                             : instance<Q8LdsGroup<kBlock>>(p.cw, p.j, p.r);
    if (!lds_chunks_ok(p, k / 16)) return hipErrorInvalidConfiguration;
    return launch_group(fn, p, g, grid, q8_lds_bytes(p.cw, p.j),
                        static_cast<int>(k / 16), stream);
}

// ---- FP16/FP32 GEMV
constexpr int64_t kGemvMaxLdsBytes = 64 * 1024;   // x staged per workgroup

bool gemv_contract_ok(int dtype, const void* w, const void* x, int64_t k) {
    const int64_t per = dtype == kF32 ? 4 : 8;     // elements per 16 bytes
    if (k % per != 0) return false;
    return (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

Plan plan_gemv(int kind, int dtype, int64_t n, int64_t k, const void* w,
               const void* x) {
    if (kind == kScalar) return scalar_plan(n, false, "");
    if (!gemv_contract_ok(dtype, w, x, k))
        return scalar_plan(n, true, "vector contract unmet (w/x 16B alignment, k % elements per 16 B)");
    const int64_t es = dtype == kF32 ? 4 : 2;
    const int64_t nchunks = k * es / 16;
    // in-row byte offsets are 32-bit in every vector kernel; row bases are
    // 64-bit only in the tiled kernel, which therefore also takes weights
    // of 4 GiB or more
    if (k * es >= (int64_t{1} << 32))
        return scalar_plan(n, true, "rows of 4 GiB or more (32-bit offsets)");
    const bool big = n * k * es >= (int64_t{1} << 32);
    Plan p;
    if (kind == kTiled || big || (nchunks + 1) * 16 > kGemvMaxLdsBytes) {
        // x staged tile by tile: 64 lanes per row, one row per wave
        p.kind = kTiled;
        p.cw = 64;
        p.j = static_cast<int>((nchunks + 63) / 64);
        p.r = 1;
        p.tile = kGemvTileJ;
        p.block = rounds_ok_512(n) ? 512 : kBlock;
        p.grid = (n + p.block / 64 - 1) / (p.block / 64);
        return p;
    }
    p.kind = kLds;
    p.cw = pow2_at_least(nchunks, 16);
    p.j = static_cast<int>((nchunks + p.cw - 1) / p.cw);
    p.r = 1;
    const int64_t waves = (n + (64 / p.cw) - 1) / (64 / p.cw);
    // 512-thread workgroups halve the x stagings: 16-20% faster at fp16
    // 4096^2 and 15% at 6144x4096 (whole rounds of CUs); with a partial
    // round among few (5120^2, 5120x13824: 2.5 rounds) 256 threads are 6-7%
    // faster; among 5+ rounds the two are level
    p.block = rounds_ok_512(waves) ? 512 : kBlock;
    p.grid = (waves + p.block / 64 - 1) / (p.block / 64);
    return p;
}

namespace {
template <typename S>
using GemvFn = void (*)(const uint4*, const uint4*, S*, int, int);

template <typename S, int NT, int JB>
GemvFn<S> gemv_instance_nt(int cw) {
    if (cw == 16) return &gemv_lds_kernel<S, 16, NT, JB>;
    if (cw == 32) return &gemv_lds_kernel<S, 32, NT, JB>;
    if (cw == 64) return &gemv_lds_kernel<S, 64, NT, JB>;
    return nullptr;
}

template <typename S, int NT>
GemvFn<S> gemv_instance_jb(int cw, int j) {
    if (j <= 2) return gemv_instance_nt<S, NT, 2>(cw);
    if (j <= 4) return gemv_instance_nt<S, NT, 4>(cw);
    return gemv_instance_nt<S, NT, kGemvBatch>(cw);
}

template <typename S>
GemvFn<S> gemv_instance(int cw, int j, int block) {
    if (block == 512) return gemv_instance_jb<S, 512>(cw, j);
    if (block == kBlock) return gemv_instance_jb<S, kBlock>(cw, j);
    return nullptr;
}

template <typename S>
hipError_t prepare_gemv_t(const Plan& p, const void* w, const void* x, void* y,
                          int64_t n, int64_t k, Launch* L) {
    if (p.kind == kScalar)
        return bind(L, gemv_scalar_kernel<S>, p.grid, p.block, 0,
                    static_cast<const S*>(w), static_cast<const S*>(x),
                    static_cast<S*>(y), k);
    const int nchunks = static_cast<int>(k * static_cast<int64_t>(sizeof(S)) / 16);
    if (p.kind == kTiled)
        return bind(L, p.block == 512 ? gemv_tiled_kernel<S, 512> : gemv_tiled_kernel<S, kBlock>,
                    p.grid, p.block, kGemvTileLds, static_cast<const uint4*>(w),
                    static_cast<const uint4*>(x), static_cast<S*>(y),
                    static_cast<int>(n), nchunks);
    const GemvFn<S> fn = gemv_instance<S>(p.cw, p.j, p.block);
    if (fn == nullptr) return hipErrorInvalidConfiguration;
    return bind(L, fn, p.grid, p.block, static_cast<uint32_t>((nchunks + 1) * 16),
                static_cast<const uint4*>(w), static_cast<const uint4*>(x),
                static_cast<S*>(y), static_cast<int>(n), nchunks);
}
}  // namespace

hipError_t prepare_gemv(const Plan& p, int dtype, const void* w, const void* x,
                        void* y, int64_t n, int64_t k, Launch* L) {
    return dtype == kF32 ? prepare_gemv_t<float>(p, w, x, y, n, k, L)
                         : prepare_gemv_t<uint16_t>(p, w, x, y, n, k, L);
}

hipError_t launch_gemv(const Plan& p, int dtype, const void* w, const void* x,
                       void* y, int64_t n, int64_t k, hipStream_t stream,
                       hipEvent_t ev0, hipEvent_t ev1) {
    Launch L;
    const hipError_t e = prepare_gemv(p, dtype, w, x, y, n, k, &L);
    return e != hipSuccess ? e : enqueue(L, stream, ev0, ev1);
}

hipError_t launch_stream_read(const void* buf, int64_t bytes, void* sink,
                              hipStream_t stream) {
    const int64_t n16 = bytes / 16;
    const int64_t grid = (n16 + kBlock - 1) / kBlock;
    return launch(stream_read_kernel, grid, kBlock, 0, stream, nullptr,
                  nullptr, static_cast<const uint4*>(buf),
                  static_cast<uint32_t*>(sink), n16, 0x9E3779B9u);
}

hipError_t launch_delay(double us, hipStream_t stream) {
    if (!(us > 0.0)) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    int khz = 0;   // wall clock rate in kHz (100 MHz on MI355X)
    e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess) return e;
    if (khz <= 0) return hipErrorInvalidValue;
    const double t = us * static_cast<double>(khz) / 1000.0;
    if (t > 1e12) return hipErrorInvalidValue;
    const uint64_t ticks = static_cast<uint64_t>(t) + 1;
    // each pass sleeps 8 x 64 cycles, several ticks: ticks + 1024 passes
    // always outlast the wait and bound it if the clock were stuck
    return launch(delay_kernel, 1, 64, 0, stream, nullptr, nullptr, ticks,
                  ticks + 1024);
}

hipError_t launch_empty(int64_t grid, int block, void* sink,
                        hipStream_t stream) {
    return launch(empty_launch_kernel, grid, block, 0, stream, nullptr,
                  nullptr, static_cast<uint32_t*>(sink), 0xFFFFFFFFu);
}

}  // namespace cq
