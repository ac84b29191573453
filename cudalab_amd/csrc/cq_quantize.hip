// On-device weight quantizers for the two GEMV operators (gfx950).
//
//   INT4, group-wise (cudalab/int4gemv_quantize.py:61-114, quantize_w + pack_q):
//     per group of 128 consecutive elements of a row
//       s32 = fp32(amax |W|) / 7
//       q   = clamp(rint_half_even(fl(W / s32)), -7, 7), q = 0 if s32 == 0
//       packed byte b of the group = (q[2b] & 15) | (q[2b+1] & 15) << 4
//       scale = fp16(s32), round to nearest even
//   INT8, per row (cudalab/qgemv_quantize.py:33-64):
//       s = fp32(amax |W_row|) / 127, q = clamp(rint(fl(W / s)), -127, 127),
//       q = 0 if s == 0, scale stored as fp32.
//
// The reference writes the scale as `amax / INT4_MAX` (a tensor divided by
// a Python number), which torch evaluates differently by device: on the CPU
// as one correctly rounded division, on a GPU as amax * fl(1 / 7) (a CPU
// scalar divisor becomes a multiplication by its float reciprocal).  The
// two differ by one fp32 step for about half of all fp16 amax values, which
// moves q at exact ties.  `rcp` selects the GPU form; otherwise the CPU
// form.  The division w / s is a tensor-by-tensor division on both devices
// (correctly rounded).
//
// The outputs are bit-identical to those definitions.  Non-finite W is not
// rejected here: a group (INT4) or row (INT8) holding NaN/Inf gets a
// non-finite scale, and no finite input can give one (|amax| <= 65504), so a
// caller checks the scale, not all of W.
//
// Fast path.  Row-major W with K % 128 == 0 is a flat sequence of groups,
// group g being elements [128 g, 128 g + 128) and scale element g.  Sixteen
// lanes (one DPP row) take one group, 8 fp16 (16 bytes) each; a wave reads
// 1 KiB of consecutive groups per load.  The amax is a max over fp16 bit
// patterns with the sign cleared (for non-negative fp16 the bit-pattern
// order is the value order), reduced across the 16 lanes with DPP row
// rotations.
//
// Quotient.  With r = v_rcp_f32(s) (at most 2 ulp from 1/s assumed, 1
// documented) the exact product p = w * r satisfies
// |p - w/s| <= |q_max| * 2^-22, and the correctly rounded quotient
// F = fl(w/s) satisfies |F - w/s| <= ulp(q_max) / 2; together below 1.9e-6
// for q_max = 7 and 3.5e-5 for 127.  m = fma(w, r, 1.5 * 2^23) rounds p once
// to an integer (RNE; the integer k sits in the low mantissa bits of m), and
// d = fma(w, r, -k) is p - k rounded once.  When |d| <= 1/2 - kNear, p is
// farther than kNear - 2^-26 from every half-integer, so no half-integer
// lies between p and F and rint(F) = k.  A lane with any element closer
// than that recomputes its 8 elements with the correctly rounded division.
//
// Packing.  bits(m) = bits(1.5 * 2^23) + k exactly (|k| < 2^22), so packed
// bytes come from integer sums of the bit patterns with the offset removed
// by one constant per word: INT4 bytes (k_lo + 8) + 16 (k_hi + 8) and INT8
// bytes k + 128 lie in [1, 255] (no carries between bytes), then an XOR of
// 0x88 / 0x80 per byte turns offset binary into two's complement.

#include <hip/hip_runtime.h>
#include <cstdint>

#include "cq_internal.h"

namespace cq {
namespace {

constexpr float kRoundMagic = 12582912.0f;          // 1.5 * 2^23
constexpr uint32_t kMagicBits = 0x4B400000u;         // bits of kRoundMagic
// word = sum_j p_j << 8j + kPack4Add with p_j = bits(m_lo) + 16 bits(m_hi)
constexpr uint32_t kPack4Add = (136u - 17u * kMagicBits) * 0x01010101u;
// word = sum_j bits(m_j) << 8j + kPack8Add
constexpr uint32_t kPack8Add = (128u - kMagicBits) * 0x01010101u;
constexpr float kNear4 = 0.5f - 0x1p-18f;           // 3.8e-6 from a half-integer
constexpr float kNear8 = 0.5f - 0x1p-13f;           // 1.2e-4 from a half-integer
constexpr int kQBlock = 256;

typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Streaming accesses: each weight byte is read once and each output byte
// written once, so loads and stores carry the nontemporal hint (measured
// 5-50% faster than plain accesses on these kernels).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void store_stream(uint32_t* p, uint32_t v) {
    __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ void store_stream(uint2* p, uint2 v) {
    const u32x2 t = {v.x, v.y};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x2*>(p));
}

__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t,
                              __builtin_elementwise_max(__builtin_bit_cast(us2, a),
                                                        __builtin_bit_cast(us2, b)));
}

// Largest |fp16| bit pattern of the 8 values in v (sign bits cleared).
__device__ __forceinline__ uint32_t amax_bits8(uint4 v) {
    const uint32_t m = 0x7FFF7FFFu;
    const uint32_t a = pk_max_u16(pk_max_u16(v.x & m, v.y & m),
                                  pk_max_u16(v.z & m, v.w & m));
    return max(a & 0xFFFFu, a >> 16);
}

// Max over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1).  Every lane of
// the row must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
    v = max(v, dpp_u32<0x128>(v));
    v = max(v, dpp_u32<0x124>(v));
    v = max(v, dpp_u32<0x122>(v));
    v = max(v, dpp_u32<0x121>(v));
    return v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
    v = row16_max(v);
    v = max(v, (uint32_t)__shfl_xor((int)v, 16));
    v = max(v, (uint32_t)__shfl_xor((int)v, 32));
    return v;
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}

__device__ __forceinline__ uint16_t f2h_bits(float f) {
    return __builtin_bit_cast(unsigned short, (_Float16)f);
}

// Scale of a group / row from its amax: the CPU form (one correctly rounded
// division) or the GPU form (product with the float reciprocal of qmax,
// folded at compile time with round-to-nearest-even).
template <int QMAX>
__device__ __forceinline__ float scale_of(float amax, bool rcp) {
    constexpr float inv = 1.0f / (float)QMAX;
    return rcp ? amax * inv : amax / (float)QMAX;
}

// The definition: clamp(rint(fl(w / s)), -qmax, qmax), 0 when s == 0.
__device__ __forceinline__ int quant_exact(float w, float s, float qmax) {
    if (s == 0.f) return 0;
    float q = rintf(w / s);
    q = fminf(fmaxf(q, -qmax), qmax);
    return (int)q;
}

// Reciprocal used by the estimate; 0 for a zero scale, so t = 0 and q = 0.
__device__ __forceinline__ float quant_rcp(float s) {
    return s == 0.f ? 0.f : __builtin_amdgcn_rcpf(s);
}

// Fast estimate for one element: bits(m) = kMagicBits + RNE(w * r), and a
// near-tie flag.
__device__ __forceinline__ uint32_t quant_fast(float w, float r, float near_lim,
                                               bool& near) {
    const float m = __builtin_fmaf(w, r, kRoundMagic);
    const float d = __builtin_fmaf(w, r, -(m - kRoundMagic));
    near |= fabsf(d) > near_lim;
    return __float_as_uint(m);
}

// The same bit form from an exact integer q.
__device__ __forceinline__ uint32_t magic_bits(int q) {
    return kMagicBits + (uint32_t)q;
}

// 8 magic-bit values (elements 0..7) -> 8 nibbles, element i at bits 4i.
__device__ __forceinline__ uint32_t pack_nibbles(const uint32_t (&b)[8]) {
    uint32_t acc = kPack4Add;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += (b[2 * j] + (b[2 * j + 1] << 4)) << (8 * j);
    return acc ^ 0x88888888u;
}

// 4 magic-bit values -> 4 int8 bytes, element i in byte i.
__device__ __forceinline__ uint32_t pack_bytes(uint32_t b0, uint32_t b1, uint32_t b2,
                                               uint32_t b3) {
    return (b0 + (b1 << 8) + (b2 << 16) + (b3 << 24) + kPack8Add) ^ 0x80808080u;
}

__device__ __forceinline__ float half_of(uint4 v, int i) {
    const uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
    return h2f((i & 1) ? (w >> 16) : (w & 0xFFFFu));
}

// 8 fp16 -> 8 nibbles (element i at bits 4i..4i+3).
__device__ __forceinline__ uint32_t int4_pack8(uint4 v, float s, float r) {
    bool near = false;
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = quant_fast(half_of(v, i), r, kNear4, near);
    if (near) {
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = magic_bits(quant_exact(half_of(v, i), s, 7.f));
    }
    return pack_nibbles(b);
}

// 8 fp16 -> 8 int8 (element i in byte i).
__device__ __forceinline__ uint2 q8_pack8(uint4 v, float s, float r) {
    bool near = false;
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = quant_fast(half_of(v, i), r, kNear8, near);
    if (near) {
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = magic_bits(quant_exact(half_of(v, i), s, 127.f));
    }
    return make_uint2(pack_bytes(b[0], b[1], b[2], b[3]), pack_bytes(b[4], b[5], b[6], b[7]));
}

// ---------------------------------------------------------------- INT4 ---
// Fast kernel: 16 lanes per group, kInt4Steps groups per 16-lane row,
// 16 * kInt4Steps groups per 256-thread workgroup.  Requires w 16-byte and
// wp 4-byte aligned.  (2 steps measured best of 1, 2, 4, 8.)
constexpr int kInt4Steps = 2;
constexpr int kInt4GroupsPerBlock = (kQBlock / 16) * kInt4Steps;

__global__ __launch_bounds__(kQBlock) void int4_quantize_kernel(
        const uint4* __restrict__ w, uint32_t* __restrict__ wp,
        uint16_t* __restrict__ scale, int64_t groups, bool rcp) {
    const int lane16 = threadIdx.x & 15;
    const int64_t g0 = (int64_t)blockIdx.x * kInt4GroupsPerBlock + (threadIdx.x >> 4);
    // Out-of-range slots (the last workgroup) re-read the last group and
    // store nothing, so every load is one unconditional 16-byte load.
    uint4 v[kInt4Steps];
#pragma unroll
    for (int u = 0; u < kInt4Steps; ++u) {
        const int64_t g = min(g0 + u * (kQBlock / 16), groups - 1);
        v[u] = load_stream(w + g * 16 + lane16);
    }
#pragma unroll
    for (int u = 0; u < kInt4Steps; ++u) {
        const int64_t g = g0 + u * (kQBlock / 16);
        const float s = scale_of<7>(h2f(row16_max(amax_bits8(v[u]))), rcp);
        const uint32_t packed = int4_pack8(v[u], s, quant_rcp(s));
        if (g < groups) {
            store_stream(wp + g * 16 + lane16, packed);
            if (lane16 == 0) scale[g] = f2h_bits(s);
        }
    }
}

// Generic kernel (any 2-byte aligned w, any wp): one wave per group, two
// elements per lane, the definition evaluated directly.
__global__ __launch_bounds__(kQBlock) void int4_quantize_generic_kernel(
        const uint16_t* __restrict__ w, uint8_t* __restrict__ wp,
        uint16_t* __restrict__ scale, int64_t groups, bool rcp) {
    const int64_t g = (int64_t)blockIdx.x * (kQBlock / 64) + (threadIdx.x >> 6);
    if (g >= groups) return;                       // uniform over the wave
    const int lane = threadIdx.x & 63;
    const uint32_t e0 = w[g * 128 + 2 * lane], e1 = w[g * 128 + 2 * lane + 1];
    const uint32_t am = wave_max(max(e0 & 0x7FFFu, e1 & 0x7FFFu));
    const float s = scale_of<7>(h2f(am), rcp);
    const uint32_t q0 = (uint32_t)quant_exact(h2f(e0), s, 7.f) & 0xFu;
    const uint32_t q1 = (uint32_t)quant_exact(h2f(e1), s, 7.f) & 0xFu;
    wp[g * 64 + lane] = (uint8_t)(q0 | (q1 << 4));
    if (lane == 0) scale[g] = f2h_bits(s);
}

// ---------------------------------------------------------------- INT8 ---
// Fast kernel: one 256-thread workgroup per row, H 16-byte chunks per
// thread held in registers between the amax and the quantize pass (rows up
// to 256 * 8 * H elements); longer rows re-read the rest (from L2).  H is
// the smallest instance that holds the row (fewer registers, more waves
// per SIMD), at most kQ8MaxHeld.  Requires k % 8 == 0, w 16-byte and wq
// 8-byte aligned.
constexpr int kQ8MaxHeld = 8;

template <int kQ8Held>
__global__ __launch_bounds__(kQBlock) void q8_quantize_kernel(
        const uint4* __restrict__ w, uint2* __restrict__ wq,
        float* __restrict__ scale, int64_t chunks, bool rcp) {
    __shared__ uint32_t red[kQBlock / 64];
    const int64_t row = blockIdx.x;
    const uint4* src = w + row * chunks;
    uint2* dst = wq + row * chunks;
    uint4 v[kQ8Held];
    uint32_t am = 0;
#pragma unroll
    for (int h = 0; h < kQ8Held; ++h) {
        const int64_t c = threadIdx.x + (int64_t)h * kQBlock;
        v[h] = c < chunks ? load_stream(src + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int h = 0; h < kQ8Held; ++h) am = max(am, amax_bits8(v[h]));
    for (int64_t c = threadIdx.x + (int64_t)kQ8Held * kQBlock; c < chunks; c += kQBlock)
        am = max(am, amax_bits8(src[c]));
    am = wave_max(am);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
    __syncthreads();
    am = max(max(red[0], red[1]), max(red[2], red[3]));
    const float s = scale_of<127>(h2f(am), rcp);
    const float r = quant_rcp(s);
    if (threadIdx.x == 0) scale[row] = s;
#pragma unroll
    for (int h = 0; h < kQ8Held; ++h) {
        const int64_t c = threadIdx.x + (int64_t)h * kQBlock;
        if (c < chunks) store_stream(dst + c, q8_pack8(v[h], s, r));
    }
    for (int64_t c = threadIdx.x + (int64_t)kQ8Held * kQBlock; c < chunks; c += kQBlock)
        dst[c] = q8_pack8(src[c], s, r);
}

// Generic kernel (any k, any 2-byte aligned w): one workgroup per row,
// element by element, the definition evaluated directly.
__global__ __launch_bounds__(kQBlock) void q8_quantize_generic_kernel(
        const uint16_t* __restrict__ w, int8_t* __restrict__ wq,
        float* __restrict__ scale, int64_t k, bool rcp) {
    __shared__ uint32_t red[kQBlock / 64];
    const int64_t row = blockIdx.x;
    const uint16_t* src = w + row * k;
    uint32_t am = 0;
    for (int64_t i = threadIdx.x; i < k; i += kQBlock) am = max(am, (uint32_t)(src[i] & 0x7FFFu));
    am = wave_max(am);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
    __syncthreads();
    am = max(max(red[0], red[1]), max(red[2], red[3]));
    const float s = scale_of<127>(h2f(am), rcp);
    if (threadIdx.x == 0) scale[row] = s;
    for (int64_t i = threadIdx.x; i < k; i += kQBlock)
        wq[row * k + i] = (int8_t)quant_exact(h2f(src[i]), s, 127.f);
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

QuantPlan plan_int4_quantize(int64_t n, int64_t k, const void* w, const void* wp) {
    QuantPlan p;
    const int64_t groups = n * (k / 128);
    p.fast = aligned(w, 16) && aligned(wp, 4);
    p.block = kQBlock;
    p.grid = p.fast ? (groups + kInt4GroupsPerBlock - 1) / kInt4GroupsPerBlock
                    : (groups + kQBlock / 64 - 1) / (kQBlock / 64);
    return p;
}

QuantPlan plan_q8_quantize(int64_t n, int64_t k, const void* w, const void* wq) {
    QuantPlan p;
    p.fast = k % 8 == 0 && aligned(w, 16) && aligned(wq, 8);
    p.block = kQBlock;
    p.grid = n;
    if (p.fast) {
        const int64_t need = (k / 8 + kQBlock - 1) / kQBlock;
        p.held = need <= 1 ? 1 : need <= 2 ? 2 : need <= 3 ? 3 : need <= 4 ? 4
               : need <= 6 ? 6 : kQ8MaxHeld;
    }
    return p;
}

hipError_t launch_int4_quantize(const QuantPlan& p, const void* w, void* wp,
                                void* scale, int64_t n, int64_t k, bool rcp,
                                hipStream_t stream) {
    const int64_t groups = n * (k / 128);
    if (p.fast)
        int4_quantize_kernel<<<dim3((unsigned)p.grid), dim3(kQBlock), 0, stream>>>(
            (const uint4*)w, (uint32_t*)wp, (uint16_t*)scale, groups, rcp);
    else
        int4_quantize_generic_kernel<<<dim3((unsigned)p.grid), dim3(kQBlock), 0, stream>>>(
            (const uint16_t*)w, (uint8_t*)wp, (uint16_t*)scale, groups, rcp);
    return hipGetLastError();
}

hipError_t launch_q8_quantize(const QuantPlan& p, const void* w, void* wq,
                              void* scale, int64_t n, int64_t k, bool rcp,
                              hipStream_t stream) {
    if (p.fast) {
        const dim3 g((unsigned)p.grid), b(kQBlock);
        const uint4* w4 = (const uint4*)w;
        uint2* q2 = (uint2*)wq;
        float* sc = (float*)scale;
        const int64_t chunks = k / 8;
        switch (p.held) {
        case 1: q8_quantize_kernel<1><<<g, b, 0, stream>>>(w4, q2, sc, chunks, rcp); break;
        case 2: q8_quantize_kernel<2><<<g, b, 0, stream>>>(w4, q2, sc, chunks, rcp); break;
        case 3: q8_quantize_kernel<3><<<g, b, 0, stream>>>(w4, q2, sc, chunks, rcp); break;
        case 4: q8_quantize_kernel<4><<<g, b, 0, stream>>>(w4, q2, sc, chunks, rcp); break;
        case 6: q8_quantize_kernel<6><<<g, b, 0, stream>>>(w4, q2, sc, chunks, rcp); break;
        default: q8_quantize_kernel<kQ8MaxHeld><<<g, b, 0, stream>>>(w4, q2, sc, chunks, rcp); break;
        }
    } else
        q8_quantize_generic_kernel<<<dim3((unsigned)p.grid), dim3(kQBlock), 0, stream>>>(
            (const uint16_t*)w, (int8_t*)wq, (float*)scale, k, rcp);
    return hipGetLastError();
}

}  // namespace cq
