/*
 * cdnaqgemv.h — C ABI of the MI355X (gfx950) weight-only quantized GEMV
 * library `libcdnaqgemv.so`.
 *
 * Two operators, both y[n] = sum_k Wdequant[n,k] * x[k] with FP32
 * accumulation and one round-to-nearest-even cast to fp16 at the end:
 *
 *   int4gemv (W4A16, group-wise INT4):
 *     w_packed u8 [n, k/2]  row-major; byte b of a row holds element 2b in
 *                           its low nibble and element 2b+1 in its high
 *                           nibble, 4-bit two's complement (-8..7)
 *     scale    f16 [n, k/128]  one scale per group of 128 elements
 *     x        f16 [k]
 *     y        f16 [n]
 *     Wdequant[n,k] = q[n,k] * float(scale[n, k/128]); k % 128 == 0.
 *
 *   qgemv (W8A16, per-row INT8):
 *     w_q   i8  [n, k] row-major
 *     scale f32 [n]
 *     x     f16 [k]
 *     y     f16 [n]
 *     Wdequant[n,k] = w_q[n,k] * scale[n]; any k >= 1.
 *
 *   gemv (FP16 / FP32, the reference's third generation):
 *     w  f16 or f32 [n, k] row-major
 *     x  same dtype [k]
 *     y  same dtype [n]
 *     y[n] = sum_k w[n,k] * x[k] in FP32, cast once to the dtype.
 *
 * Plus the on-device quantizers that produce the first two operators'
 * weights from fp16 W (cq_int4_quantize, cq_q8_quantize).
 *
 * All pointers are device pointers on the current HIP device; `stream` is a
 * hipStream_t (NULL = the null stream).  Calls are asynchronous: a kernel is
 * enqueued and the call returns.  The library never allocates device memory
 * on these paths and keeps no state between calls.
 *
 * Vector contract (checked on the host before every launch): the vectorized
 * kernels need w and x 16-byte aligned and k % 32 == 0 (int4gemv),
 * k % 16 == 0 (qgemv), k % 8 == 0 (gemv fp16) or k % 4 == 0 (gemv fp32).  Inputs that miss it are never rejected: they run on
 * the scalar kernel of the `*_baseline` variant, so their output is
 * bit-identical to that variant's.
 *
 * Errors: every entry point returns a CQ_* status; on error nothing was
 * launched (or, for CQ_ERR_HIP, the HIP runtime refused the launch) and
 * cq_last_error() returns a message for the calling thread.  Metadata
 * validation with the reference's messages (dtype, contiguity, device) is
 * the Python layer's job; this layer re-checks only what it needs to launch
 * safely (non-null pointers, positive sizes, k % 128 for int4gemv, outputs
 * that share no byte with the inputs).
 *
 * Any k: rows longer than 16384 elements (int4gemv, qgemv) or whose x
 * exceeds 64 KiB (gemv), and weights of 4 GiB or more, run K-tiled
 * vectorized kernels on the LDS variants (describe reports kernel=tiled).
 */
#ifndef CDNAQGEMV_H
#define CDNAQGEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define CQ_OK                   0
#define CQ_ERR_UNKNOWN_VARIANT  1
#define CQ_ERR_INVALID_ARG      2
#define CQ_ERR_HIP              3
#define CQ_ERR_BUFFER_TOO_SMALL 4

/* operator ids (the timing, list and describe entry points take these;
 * gemv has one id per dtype and one shared variant registry) */
#define CQ_OP_INT4GEMV 0
#define CQ_OP_QGEMV    1
#define CQ_OP_GEMV_F16 2
#define CQ_OP_GEMV_F32 3

/* gemv element types */
#define CQ_DTYPE_F16 0
#define CQ_DTYPE_F32 1

/* quantizer scale forms (cq_int4_quantize, cq_q8_quantize): the reference
 * computes the scale as `amax / qmax` in torch, which is one correctly
 * rounded division for a CPU tensor and amax * fl(1 / qmax) for a GPU
 * tensor (torch applies a CPU-scalar divisor as its reciprocal) */
#define CQ_SCALE_DIV 0   /* amax / qmax: the reference run on the CPU */
#define CQ_SCALE_RCP 1   /* amax * fl(1/qmax): the reference run on a GPU */

/* variant list selectors */
#define CQ_LIST_NORMAL      0
#define CQ_LIST_ALL         1
#define CQ_LIST_QUARANTINED 2
#define CQ_LIST_ALIASES     3

/*
 * One INT4 W4A16 GEMV launch: y = (unpack(w_packed) * scale) @ x.
 * Replaces the variant entry `int4gemv_fn_t`
 * (kernels/int4gemv/int4gemv_common.h:89-92) behind
 * `int4gemv_forward` / `int4gemv_forward_into`
 * (kernels/int4gemv/bindings.cpp:145-176).  `variant` is a name from
 * cq_variants(CQ_OP_INT4GEMV, ...), e.g. "int4gemv_baseline".
 * For this and every other launching entry point, y must not share a byte
 * with w, scale or x of the same call (CQ_ERR_INVALID_ARG, nothing
 * launched): workgroups write y while others still read the inputs.
 */
int cq_int4gemv(const char* variant, const void* w_packed, const void* scale,
                const void* x, void* y, int64_t n, int64_t k, void* stream);

/*
 * One INT8 W8A16 GEMV launch: y = (w_q * scale[:,None]) @ x.
 * Replaces `qgemv_fn_t` (kernels/qgemv/qgemv_common.h:64-67) behind
 * `qgemv_forward` / `qgemv_forward_into`
 * (kernels/qgemv/bindings.cpp:140-173).
 */
int cq_qgemv(const char* variant, const void* w_q, const void* scale,
             const void* x, void* y, int64_t n, int64_t k, void* stream);

/*
 * One FP16 or FP32 GEMV launch: y = w @ x, FP32 accumulation, y in the
 * dtype of w (dtype = CQ_DTYPE_F16 or CQ_DTYPE_F32).  Replaces `gemv_fn_t`
 * (kernels/gemv/gemv_common.h:53-55) behind `gemv_forward` /
 * `gemv_forward_into` (kernels/gemv/bindings.cpp:137-190).
 */
int cq_gemv(const char* variant, int dtype, const void* w, const void* x,
            void* y, int64_t n, int64_t k, void* stream);

/* One problem of a grouped call: device pointers and its row count. */
typedef struct cq_gemv_problem {
    const void* w;      /* w_packed (int4gemv) or w_q (qgemv) */
    const void* scale;
    const void* x;
    void* y;
    int64_t n;
} cq_gemv_problem_t;

/*
 * Grouped GEMV: n_problems independent problems of one operator that share
 * k, enqueued with as few launches as possible (one launch per 8 problems
 * for the CDNA4 LDS variants; the other variants, and any 8-problem batch
 * in which a problem misses the vector contract, launch problem by
 * problem).  Each y is bit-identical to a cq_int4gemv / cq_qgemv call of
 * the same variant on the same problem.  Every problem is checked as a
 * single call would be before anything is launched.  The problems run at
 * the same time, so no problem's y may share a byte with another problem's
 * w, scale, x or y (CQ_ERR_INVALID_ARG naming both problems); inputs may be
 * shared (q/k/v read one x).  No counterpart in the
 * reference (its variants launch one problem at a time): it serves decode
 * steps whose projections are independent (q/k/v; gate/up) and pays the
 * per-launch cost once per batch.
 */
int cq_int4gemv_grouped(const char* variant, const cq_gemv_problem_t* problems,
                        int64_t n_problems, int64_t k, void* stream);
int cq_qgemv_grouped(const char* variant, const cq_gemv_problem_t* problems,
                     int64_t n_problems, int64_t k, void* stream);

/*
 * On-device INT4 quantize + pack of fp16 w [n, k] (k % 128 == 0) into
 * w_packed uint8 [n, k/2] and scale fp16 [n, k/128]: per group of 128,
 * s = fp32 amax / 7 in the form `scale_mode` names (CQ_SCALE_DIV or
 * CQ_SCALE_RCP), q = clamp(rint_half_even(w / s), -7, 7) (0 for a zero
 * group), element 2b in the low nibble of byte b, scale = fp16(s).
 * Bit-identical to `quantize_w` + `pack_q`
 * (cudalab/int4gemv_quantize.py:61-114), which the reference runs as torch
 * ops, on the CPU (CQ_SCALE_DIV) or on a GPU (CQ_SCALE_RCP).  Asynchronous
 * on `stream`.  NaN/Inf in w is not rejected: the scale of every group
 * holding one is non-finite, and finite w never gives a non-finite scale,
 * so a caller checks the scale.  w, w_packed and scale must not overlap
 * (CQ_ERR_INVALID_ARG; the same holds for cq_q8_quantize).
 */
int cq_int4_quantize(const void* w, void* w_packed, void* scale, int64_t n,
                     int64_t k, int scale_mode, void* stream);

/*
 * On-device INT8 quantize of fp16 w [n, k] (any k >= 1) into w_q int8
 * [n, k] and scale fp32 [n]: s = fp32 row amax / 127 (form per
 * `scale_mode`), q = clamp(rint_half_even(w / s), -127, 127), 0 for a zero
 * row.  Bit-identical to `quantize_w` (cudalab/qgemv_quantize.py:33-64) on
 * the CPU (CQ_SCALE_DIV) or a GPU (CQ_SCALE_RCP).  NaN/Inf as for
 * cq_int4_quantize (per row).
 */
int cq_q8_quantize(const void* w, void* w_q, void* scale, int64_t n, int64_t k,
                   int scale_mode, void* stream);

/*
 * 1 if the quantizer of `op` (CQ_OP_INT4GEMV or CQ_OP_QGEMV) takes its
 * vectorized kernel for these pointers and sizes (w 16-byte aligned,
 * output 4-byte (INT4) or 8-byte (INT8) aligned, k % 8 == 0 for INT8),
 * 0 if it takes the element-wise kernel (same results), -1 for another op.
 * No reference counterpart (the reference quantizes with torch ops).
 */
int cq_quantize_vectorized(int op, const void* w, const void* out, int64_t n,
                           int64_t k);

/* Result of cq_native_timing; all times are per launch, microseconds. */
typedef struct cq_timing {
    int64_t warmup;
    int64_t n_windows;
    int64_t launches_per_window;
    double median_us;
    double min_us;
    double max_us;
    double mean_us;
} cq_timing_t;

/*
 * Native kernel-loop timing: `warmup` untimed launches, then `n_windows`
 * windows of `launches_per_window` back-to-back launches, each window
 * bracketed by HIP events on `stream`; window_us[i] (caller-owned, length
 * n_windows, may be NULL) receives window time / launches.  Replaces
 * `int4gemv_native_timing` (kernels/int4gemv/bindings.cpp:180-253) and
 * `qgemv_native_timing` (kernels/qgemv/bindings.cpp:175-249).  Synchronizes
 * the stream.
 */
int cq_native_timing(int op, const char* variant, const void* w,
                     const void* scale, const void* x, void* y, int64_t n,
                     int64_t k, void* stream, int64_t warmup,
                     int64_t n_windows, int64_t launches_per_window,
                     double* window_us, cq_timing_t* out);

/*
 * The timing loops below share one window.  Untimed launches run first,
 * until both `warmup` launches and `burn_ms` milliseconds of wall-clock
 * time have passed (clocks and power settle; the reference's measure_block
 * burns at least 150 launches and 300 ms, cudalab/evaluator/bench.py:294-300),
 * and the stream is synchronized.  Then, if delay_us > 0, a bounded
 * on-device wait of about delay_us microseconds is queued (one wave, no
 * memory work, bounded by an iteration count as well as by the clock), so
 * that the host can enqueue the timed launches before the GPU reaches
 * them; then the start event, the `n_launches` timed launches and the stop
 * event.  *total_us receives the event time of the window.  The wait lies
 * before the start event, outside the window.  Each call synchronizes the
 * stream.  burn_ms must lie in [0, 600000] and delay_us in [0, 1e6].
 */

/*
 * Rotating-pool timing for HBM-cold ("streaming") measurement: launch i
 * uses set (i % n_sets) of the caller's arrays w[], scale[], x[], y[]
 * (the rotation runs on through warm-up and window).  *host_us (may be
 * NULL) receives the host time spent enqueuing the window: when it reaches
 * *total_us the window was bound by submission, not by the GPU.  If
 * kernel_us (caller-owned, length n_launches) is non-NULL, every timed
 * launch also carries start/stop events on the dispatch itself
 * (hipExtLaunchKernel) and kernel_us[i] receives their difference; on
 * MI355X these per-dispatch events read about 4 us even for an empty
 * kernel, so they are only meaningful for long kernels.  No counterpart in
 * the reference's C++ layer: it restates the x/out rotation of
 * `BenchPool` + `measure_block`
 * (cudalab/evaluator/bench.py:197-309) in native code, with W rotated too.
 */
int cq_pool_timing(int op, const char* variant, const void* const* w,
                   const void* const* scale, const void* const* x,
                   void* const* y, int64_t n_sets, int64_t n, int64_t k,
                   void* stream, int64_t warmup, double burn_ms,
                   double delay_us, int64_t n_launches, float* kernel_us,
                   double* total_us, double* host_us);

/*
 * Read-only ceiling: a plain streaming-read kernel, launch i reading
 * `bytes` (a multiple of 16) from bufs[i % n_bufs] (16-byte aligned device
 * buffers), in the window described above.  `sink` is a device buffer of
 * at least 4 bytes that the kernel may write.  No counterpart in the
 * reference: it measures the bandwidth one launch can reach for a given
 * byte count on this device (the ceiling a GEMV call of the same bytes is
 * compared against).
 */
int cq_read_ceiling(const void* const* bufs, int64_t n_bufs, int64_t bytes,
                    void* sink, void* stream, int64_t warmup, double burn_ms,
                    double delay_us, int64_t n_launches, double* total_us);

/*
 * Launch floor: a kernel that does no memory work, `grid` workgroups
 * (1..INT_MAX) of `block` threads (1..1024), in the window described
 * above.  `sink` is a device buffer of at least 4 bytes (never written).
 * No counterpart in the reference: it measures what one dispatch of a
 * GEMV's launch shape costs on this device before any kernel body runs.
 */
int cq_launch_floor(int64_t grid, int block, void* sink, void* stream,
                    int64_t warmup, double burn_ms, double delay_us,
                    int64_t n_launches, double* total_us);

/*
 * Wave timeline of the INT4 GEMV (a diagnostic; no counterpart in the
 * reference: it shows where the time of one call goes).  The sets and the
 * window are those of cq_pool_timing (op CQ_OP_INT4GEMV); every launch,
 * untimed ones included, runs a copy of the LDS kernel that `variant` plans
 * for (n, k) -- the same arithmetic, launch shape and y -- which stamps each
 * of its `waves` waves (*waves_out = grid * block / 64).  Launch i writes 8
 * words per wave at stamps[((i % n_launches) * waves + wave) * 8]: the wall
 * clock at the wave's start, after its x barrier, after its first and its
 * last weight chunk are summed, after its y stores are issued, then the
 * wave's hardware CU id and two zero words.  Every slot is last written by
 * one of the n_launches timed launches; their order follows from the
 * stamps.  `stamps` is device memory of `stamps_words` (at least
 * n_launches * waves * 8) 64-bit words.  *ticks_per_us is the clock's rate,
 * *total_us the window's event time.  CQ_ERR_INVALID_ARG when a set's plan
 * is not the LDS kernel (the scalar or K-tiled kernels are not covered) or
 * when the stamps share a byte with an operand of a set.
 */
int cq_int4_timeline(const char* variant, const void* const* w,
                     const void* const* scale, const void* const* x,
                     void* const* y, int64_t n_sets, int64_t n, int64_t k,
                     void* stream, int64_t warmup, double burn_ms,
                     double delay_us, int64_t n_launches, uint64_t* stamps,
                     int64_t stamps_words, int64_t* waves_out,
                     double* ticks_per_us, double* total_us);

/*
 * Variant names of `op`, sorted, '\n'-separated, NUL-terminated, written to
 * buf (capacity cap).  which = CQ_LIST_NORMAL (dispatchable),
 * CQ_LIST_ALL (also quarantined), CQ_LIST_QUARANTINED, or CQ_LIST_ALIASES
 * ("alias=target" lines: the reference's variant names accepted as
 * aliases).  Returns the length needed including the NUL (> 0), or a
 * negative CQ_* status; if cap is too small nothing is written past cap.
 * Replaces `int4gemv_variant_list` / `_all_variant_list` /
 * `_quarantined_variant_list` (kernels/int4gemv/bindings.cpp:258-285) and
 * the qgemv equivalents (kernels/qgemv/bindings.cpp:251-278).
 */
int cq_variants(int op, int which, char* buf, size_t cap);

/*
 * Host predicate of the vector contract: 1 if the vectorized kernels of
 * `op` may run on (w, x, k), else 0.  Replaces `int4gemv_vec_contract_ok`
 * (kernels/int4gemv/int4gemv_common.h:115-121) and `qgemv_vec_contract_ok`
 * (kernels/qgemv/qgemv_common.h:90-95).
 */
int cq_vec_contract_ok(int op, const void* w, const void* x, int64_t k);

/*
 * Describes, without launching anything, the kernel and launch shape that
 * cq_int4gemv / cq_qgemv would use for (variant, n, k, w, x): a one-line
 * "key=value ..." string with the keys variant, kernel (scalar, wave, lds
 * or tiled), cw (lanes per row segment), j (chunks per lane), r (rows per
 * lane), tile (chunks per lane per tile of the K-tiled kernels, else 0),
 * block, grid, lds (dynamic LDS bytes per workgroup of that launch),
 * fallback and, last, why (free text, "-" if none).  No
 * counterpart in the reference (its variants
 * have fixed shapes); exposed for tests and tuning records.  Returns the
 * needed length including the NUL, or a negative CQ_* status.
 */
int cq_describe_launch(int op, const char* variant, int64_t n, int64_t k,
                       const void* w, const void* x, char* buf, size_t cap);

/*
 * A launch resolved ahead of time: opaque plain data, no resources held.
 * Zero-initialised or damaged records are refused by cq_launch_prepared.
 */
typedef struct cq_prepared {
    uint64_t opaque[12];
} cq_prepared_t;

/*
 * Runs every check and the plan of one cq_int4gemv (op = CQ_OP_INT4GEMV),
 * cq_qgemv (CQ_OP_QGEMV) or cq_gemv (CQ_OP_GEMV_F16 / CQ_OP_GEMV_F32;
 * `scale` ignored) call, with the same arguments and the same status and
 * cq_last_error() on failure, and stores the resolved launch (kernel
 * instance, grid, block, LDS bytes, arguments) in *out instead of
 * enqueueing it.  On failure *out is zeroed.  Nothing is launched and no
 * GPU call is made.
 *
 * No counterpart in the reference: its pybind modules validate and launch
 * in one call (kernels/int4gemv/bindings.cpp:145-176,
 * kernels/qgemv/bindings.cpp:140-173).  For callers that issue the same
 * GEMV on the same buffers many times from the host (a decode loop, an
 * eager Python API that caches per operand set), so that the checks are
 * paid once.
 */
int cq_prepare(int op, const char* variant, const void* w, const void* scale,
               const void* x, void* y, int64_t n, int64_t k, cq_prepared_t* out);

/*
 * Enqueues a prepared launch on `stream` (NULL = the default stream).  The
 * stream must belong to the device that was current at cq_prepare, and the
 * buffers named there must still be allocated: the record holds raw device
 * pointers and is not re-validated beyond its integrity check
 * (CQ_ERR_INVALID_ARG for a record cq_prepare did not fill).  Results are
 * bit-identical to the direct call.  Returns CQ_OK or CQ_ERR_HIP.
 */
int cq_launch_prepared(const cq_prepared_t* prepared, void* stream);

/*
 * Message of the last failed call on this thread ("" if none).  Replaces
 * the TORCH_CHECK error text that the reference's pybind layer raised.
 */
const char* cq_last_error(void);

/* Library version string. */
const char* cq_version(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* CDNAQGEMV_H */
