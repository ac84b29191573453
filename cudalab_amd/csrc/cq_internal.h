// Internal interface between the C ABI layer (cq_capi.cpp) and the gfx950
// kernels (cq_kernels.hip).  Not installed; the public surface is
// include/cdnaqgemv.h.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

namespace cq {

// Kernel families.  kScalar is the single scalar source shared by the
// *_baseline variants and by every fallback, so a fallback is bit-identical
// to the baseline on the same input.  kWave is the CDNA4 wave64 kernel with
// x in registers, kLds the one that stages x once per workgroup in LDS, and
// kTiled the LDS kernel for rows of any length: one row per wave, x staged
// tile by tile.
enum Kind : int { kScalar = 0, kWave = 1, kLds = 2, kTiled = 3 };

// Largest reduction length (elements) the wave and LDS kernels take: 16384
// = 8 chunks per lane (INT4) or 16 (INT8) held at once.  Beyond it the LDS
// variants run the tiled kernel and the wave variants the scalar kernel.
constexpr int64_t kMaxWaveK = 16384;

// A resolved launch: which kernel instance and with what shape.
struct Plan {
    int kind = kScalar;   // Kind
    int cw = 0;           // lanes per row segment (16, 32 or 64)
    int j = 0;            // chunks held per lane (x registers)
    int r = 0;            // rows per lane
    int tile = 0;         // chunks per lane per tile (K-tiled kernels), else 0
    int block = 0;        // threads per workgroup
    int64_t grid = 0;     // workgroups
    bool fallback = false;  // requested a wave variant, got the scalar kernel
    std::string why;      // reason for a fallback ("" otherwise)
};

// Launch-shape selection.  `rows` = 0 lets the library pick rows per lane
// from its tuning table; otherwise it is the requested rows per lane
// (clamped to what the register budget of the instance allows).
Plan plan_int4(int kind, int rows, int64_t n, int64_t k, const void* w,
               const void* x);
Plan plan_q8(int kind, int rows, int64_t n, int64_t k, const void* w,
             const void* x);

bool int4_contract_ok(const void* w, const void* x, int64_t k);
bool q8_contract_ok(const void* w, const void* x, int64_t k);

// A launch resolved to its kernel instance, shape and arguments: plain data
// holding no pointer into the library's state (the kernel address is the
// instance's host-side handle), built once and enqueued any number of times,
// on any stream of the device whose operands it names.  Each kernel argument
// sits in its own 8-byte slot.
constexpr int kMaxLaunchArgs = 6;
struct Launch {
    const void* fn = nullptr;
    uint32_t grid = 0, block = 0, shmem = 0, nargs = 0;
    uint64_t args[kMaxLaunchArgs] = {};
};

// Resolve `plan` on the given operands into a Launch (no GPU call).
hipError_t prepare_int4(const Plan& plan, const void* w, const void* scale,
                        const void* x, void* y, int64_t n, int64_t k, Launch* out);
hipError_t prepare_q8(const Plan& plan, const void* w, const void* scale,
                      const void* x, void* y, int64_t n, int64_t k, Launch* out);

// Enqueue a resolved launch on `stream`; ev0/ev1 as below.
hipError_t enqueue(const Launch& launch, hipStream_t stream, hipEvent_t ev0,
                   hipEvent_t ev1);

// Enqueue one launch of `plan` on `stream`.  ev0/ev1, when non-null, are
// attached to the dispatch itself (start/stop of the kernel).
hipError_t launch_int4(const Plan& plan, const void* w, const void* scale,
                       const void* x, void* y, int64_t n, int64_t k,
                       hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1);
hipError_t launch_q8(const Plan& plan, const void* w, const void* scale,
                     const void* x, void* y, int64_t n, int64_t k,
                     hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1);

// The timeline diagnostic: one launch of an INT4 LDS plan (kind kLds only)
// through the stamped copy of its kernel, which writes 8 words per wave to
// `stamps` (waves = grid * block / 64).
hipError_t launch_int4_stamped(const Plan& plan, const void* w, const void* scale,
                               const void* x, void* y, int64_t n, int64_t k,
                               uint64_t* stamps, hipStream_t stream);

// Grouped launches: up to kMaxGroup independent problems of one k in one
// launch of the LDS kernels.
constexpr int kMaxGroup = 8;

struct GroupProblem {
    const void* w;
    const void* scale;
    const void* x;
    void* y;
    int64_t n;
};

// Plan of a grouped launch of `count` (1..kMaxGroup) problems.  Kind kLds
// when every problem meets the vector contract and the LDS kernels' size
// limits; otherwise kind kScalar with `fallback` set, meaning "launch the
// problems one by one" (each then gets its own plan).  `rows` as above.
Plan plan_int4_group(int rows, const GroupProblem* probs, int count, int64_t k);
Plan plan_q8_group(int rows, const GroupProblem* probs, int count, int64_t k);
hipError_t launch_int4_group(const Plan& plan, const GroupProblem* probs,
                             int count, int64_t k, hipStream_t stream);
hipError_t launch_q8_group(const Plan& plan, const GroupProblem* probs,
                           int count, int64_t k, hipStream_t stream);

// FP16/FP32 GEMV (the reference's kernels/gemv): element type of W, x, y.
enum Dtype : int { kF16 = 0, kF32 = 1 };
bool gemv_contract_ok(int dtype, const void* w, const void* x, int64_t k);
Plan plan_gemv(int kind, int dtype, int64_t n, int64_t k, const void* w,
               const void* x);
hipError_t prepare_gemv(const Plan& plan, int dtype, const void* w,
                        const void* x, void* y, int64_t n, int64_t k, Launch* out);
hipError_t launch_gemv(const Plan& plan, int dtype, const void* w,
                       const void* x, void* y, int64_t n, int64_t k,
                       hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1);

// On-device weight quantizers (INT4 group-wise with packing, INT8 per row).
// `fast` selects the vectorized kernel (alignment and k permitting); the
// generic kernel evaluates the same definition element by element.
struct QuantPlan {
    bool fast = false;
    int block = 0;
    int64_t grid = 0;
    int held = 0;   // INT8 fast kernel: 16-byte chunks per thread in registers
};
QuantPlan plan_int4_quantize(int64_t n, int64_t k, const void* w, const void* wp);
QuantPlan plan_q8_quantize(int64_t n, int64_t k, const void* w, const void* wq);
// `rcp`: scale = amax * fl(1/qmax) (torch's form on a GPU) instead of
// amax / qmax (torch's form on the CPU).
hipError_t launch_int4_quantize(const QuantPlan& p, const void* w, void* wp,
                                void* scale, int64_t n, int64_t k, bool rcp,
                                hipStream_t stream);
hipError_t launch_q8_quantize(const QuantPlan& p, const void* w, void* wq,
                              void* scale, int64_t n, int64_t k, bool rcp,
                              hipStream_t stream);

// Plain streaming read of `bytes` (a multiple of 16) from `buf`: the
// bandwidth ceiling of one launch reading that many bytes.
hipError_t launch_stream_read(const void* buf, int64_t bytes, void* sink,
                              hipStream_t stream);

// A bounded on-device wait of about `us` microseconds (one wave, no
// memory work), queued ahead of a timed window so that the host can
// enqueue the window's launches before the GPU reaches them.  No launch
// when us <= 0.
hipError_t launch_delay(double us, hipStream_t stream);

// One launch of a kernel with no memory work, `grid` workgroups of `block`
// threads (1..1024): the per-dispatch cost of that launch shape.
hipError_t launch_empty(int64_t grid, int block, void* sink,
                        hipStream_t stream);

}  // namespace cq
