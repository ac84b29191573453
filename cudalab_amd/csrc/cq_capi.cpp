// C ABI of libcdnaqgemv.so (declared in include/cdnaqgemv.h).
//
// The variant registry, the launch entry points and the two timing loops.
// The registry is a constant table (no static-initialisation registrars):
// names are unique by construction and lists are sorted on output, which is
// the contract of the reference's registry
// (kernels/int4gemv/bindings.cpp:41-56,136-142,258-285).
//
// Validation here is limited to what a safe launch needs.  Dtype,
// contiguity, device and shape-consistency checks with the reference's
// messages live in the Python layer (cudalab_amd/ext.py), which sees the
// tensors; this layer sees only pointers and sizes.

#include "cdnaqgemv.h"
#include "cq_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

struct Variant {
    const char* name;
    int op;
    int kind;         // cq::Kind
    int rows;         // rows per lane; 0 = library default per shape
    bool quarantined; // registered but hidden from the normal list
};

// Quarantine is kept as a mechanism (a variant can be listed here with
// quarantined = true) and is empty today, as in the reference
// (kernels/int4gemv/bindings.cpp:46-56).
constexpr Variant kVariants[] = {
    {"int4gemv_baseline", CQ_OP_INT4GEMV, cq::kScalar, 0, false},
    {"int4gemv_cdna4", CQ_OP_INT4GEMV, cq::kLds, 0, false},
    {"int4gemv_wave_r1", CQ_OP_INT4GEMV, cq::kWave, 1, false},
    {"int4gemv_wave_r2", CQ_OP_INT4GEMV, cq::kWave, 2, false},
    {"int4gemv_wave_r4", CQ_OP_INT4GEMV, cq::kWave, 4, false},
    {"int4gemv_lds_r1", CQ_OP_INT4GEMV, cq::kLds, 1, false},
    {"int4gemv_lds_r2", CQ_OP_INT4GEMV, cq::kLds, 2, false},
    {"int4gemv_lds_r4", CQ_OP_INT4GEMV, cq::kLds, 4, false},
    {"int4gemv_lds_tiled", CQ_OP_INT4GEMV, cq::kTiled, 0, false},
    {"qgemv_baseline", CQ_OP_QGEMV, cq::kScalar, 0, false},
    {"qgemv_cdna4", CQ_OP_QGEMV, cq::kLds, 0, false},
    {"qgemv_wave_r1", CQ_OP_QGEMV, cq::kWave, 1, false},
    {"qgemv_wave_r2", CQ_OP_QGEMV, cq::kWave, 2, false},
    {"qgemv_wave_r4", CQ_OP_QGEMV, cq::kWave, 4, false},
    {"qgemv_lds_r1", CQ_OP_QGEMV, cq::kLds, 1, false},
    {"qgemv_lds_r2", CQ_OP_QGEMV, cq::kLds, 2, false},
    {"qgemv_lds_r4", CQ_OP_QGEMV, cq::kLds, 4, false},
    {"qgemv_lds_tiled", CQ_OP_QGEMV, cq::kTiled, 0, false},
    // gemv: one registry for both dtypes (listed under CQ_OP_GEMV_F16).
    // gemv_splitk4 keeps the reference's quarantined name for callers that
    // name it explicitly (kernels/gemv/bindings.cpp:50-80); it runs the
    // scalar kernel here: a split-K GEMV needs a cross-workgroup workspace,
    // which is what the reference quarantined it for.
    {"gemv_baseline", CQ_OP_GEMV_F16, cq::kScalar, 0, false},
    {"gemv_cdna4", CQ_OP_GEMV_F16, cq::kLds, 0, false},
    {"gemv_lds_tiled", CQ_OP_GEMV_F16, cq::kTiled, 0, false},
    {"gemv_splitk4", CQ_OP_GEMV_F16, cq::kScalar, 0, true},
};

// The reference's vectorized variant names, accepted so that callers with
// a hard-coded name keep working (scripts/gen3_native_timing.py:59,66 uses
// qgemv_vec16_row).  Every one of them had the same operator contract,
// alignment contract and scalar fallback; they resolve to the CDNA4
// incumbent of their operator.
struct Alias {
    const char* alias;
    const char* target;
    int op;
};
constexpr Alias kAliases[] = {
    {"int4gemv_vec16_row", "int4gemv_cdna4", CQ_OP_INT4GEMV},
    {"int4gemv_rowtile4", "int4gemv_cdna4", CQ_OP_INT4GEMV},
    {"int4gemv_rowtile8", "int4gemv_cdna4", CQ_OP_INT4GEMV},
    {"int4gemv_rowtile4_hx", "int4gemv_cdna4", CQ_OP_INT4GEMV},
    {"qgemv_vec16_row", "qgemv_cdna4", CQ_OP_QGEMV},
    {"qgemv_vec16_scale", "qgemv_cdna4", CQ_OP_QGEMV},
    {"qgemv_warp_vec16", "qgemv_cdna4", CQ_OP_QGEMV},
    {"qgemv_warp_vec16_ilp4", "qgemv_cdna4", CQ_OP_QGEMV},
    {"gemv_vec4_row", "gemv_cdna4", CQ_OP_GEMV_F16},
    {"gemv_warp_vec4", "gemv_cdna4", CQ_OP_GEMV_F16},
};

bool valid_op(int op) {
    return op == CQ_OP_INT4GEMV || op == CQ_OP_QGEMV || op == CQ_OP_GEMV_F16 ||
           op == CQ_OP_GEMV_F32;
}

bool is_gemv(int op) { return op == CQ_OP_GEMV_F16 || op == CQ_OP_GEMV_F32; }

// Registry key of an operator id: both gemv dtypes share one registry.
int family(int op) { return op == CQ_OP_GEMV_F32 ? CQ_OP_GEMV_F16 : op; }

const char* op_name(int op) {
    if (op == CQ_OP_INT4GEMV) return "int4gemv";
    if (op == CQ_OP_QGEMV) return "qgemv";
    return is_gemv(op) ? "gemv" : "?";
}

const Variant* find_variant(int op, const char* name) {
    if (name == nullptr) return nullptr;
    const int f = family(op);
    for (const Alias& a : kAliases)
        if (a.op == f && std::strcmp(a.alias, name) == 0) name = a.target;
    for (const Variant& v : kVariants)
        if (v.op == f && std::strcmp(v.name, name) == 0) return &v;
    return nullptr;
}

// Byte ranges of one problem's operands (w, scale, x, y), for the overlap
// checks.  A kernel reads w, scale and x while other workgroups already
// write y, so y must not share a byte with them; in a grouped launch no
// problem's y may share a byte with any operand of another problem either.
// gemv has no scale (empty range).  Sizes are computed in 128 bits: n and
// k are at most 2^31 - 1, so no product overflows.
struct Span {
    unsigned __int128 lo = 0, hi = 0;
};

bool overlaps(const Span& a, const Span& b) {
    return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi;
}

struct Operands {
    Span w, scale, x, y;
};

Operands operand_spans(int op, const void* w, const void* scale, const void* x,
                       const void* y, int64_t n, int64_t k) {
    using U = unsigned __int128;
    const U un = static_cast<U>(n), uk = static_cast<U>(k);
    U wb, sb = 0, xe = 2, ye = 2;
    if (op == CQ_OP_INT4GEMV) {
        wb = un * uk / 2;
        sb = un * (uk / 128) * 2;
    } else if (op == CQ_OP_QGEMV) {
        wb = un * uk;
        sb = un * 4;
    } else {
        xe = ye = op == CQ_OP_GEMV_F32 ? 4 : 2;
        wb = un * uk * xe;
    }
    auto span = [](const void* p, U bytes) {
        Span r;
        r.lo = reinterpret_cast<uintptr_t>(p);
        r.hi = r.lo + bytes;
        return r;
    };
    return {span(w, wb), span(scale, scale != nullptr ? sb : 0), span(x, uk * xe),
            span(y, un * ye)};
}

// Shared pre-launch checks of both operators.  Returns CQ_OK or a status
// with the message set.
int check_call(int op, const char* variant, const Variant** out,
               const void* w, const void* scale, const void* x,
               const void* y, int64_t n, int64_t k) {
    if (!valid_op(op))
        return fail(CQ_ERR_INVALID_ARG, "unknown operator id " + std::to_string(op));
    if (variant == nullptr) return fail(CQ_ERR_INVALID_ARG, "variant name is NULL");
    const Variant* v = find_variant(op, variant);
    if (v == nullptr)
        return fail(CQ_ERR_UNKNOWN_VARIANT,
                    std::string("unknown ") + op_name(op) + " variant '" + variant + "'");
    // gemv has no scale (the argument is ignored and may be NULL)
    if (w == nullptr || (scale == nullptr && !is_gemv(op)) || x == nullptr ||
        y == nullptr)
        return fail(CQ_ERR_INVALID_ARG, "null device pointer");
    if (n <= 0 || n > INT_MAX)
        return fail(CQ_ERR_INVALID_ARG, "n must be in [1, 2^31-1], got " + std::to_string(n));
    if (k <= 0 || k > INT_MAX)
        return fail(CQ_ERR_INVALID_ARG, "k must be in [1, 2^31-1], got " + std::to_string(k));
    if (op == CQ_OP_INT4GEMV && k % 128 != 0)
        return fail(CQ_ERR_INVALID_ARG,
                    "k must be divisible by 128 (group_size=128), got " + std::to_string(k));
    *out = v;
    return CQ_OK;
}

// The output of a call must not share a byte with its inputs.  Run after
// check_call by every entry point that launches.
int check_disjoint(int op, const void* w, const void* scale, const void* x,
                   const void* y, int64_t n, int64_t k) {
    const Operands o = operand_spans(op, w, is_gemv(op) ? nullptr : scale, x, y, n, k);
    if (overlaps(o.y, o.w) || overlaps(o.y, o.scale) || overlaps(o.y, o.x))
        return fail(CQ_ERR_INVALID_ARG,
                    "output y overlaps an input (w, scale or x) of the same call");
    return CQ_OK;
}

// check_call, then check_disjoint.
int check_launch(int op, const char* variant, const Variant** out,
                 const void* w, const void* scale, const void* x,
                 const void* y, int64_t n, int64_t k) {
    const int st = check_call(op, variant, out, w, scale, x, y, n, k);
    return st != CQ_OK ? st : check_disjoint(op, w, scale, x, y, n, k);
}

int gemv_dtype(int op) { return op == CQ_OP_GEMV_F32 ? cq::kF32 : cq::kF16; }

cq::Plan make_plan(int op, const Variant& v, int64_t n, int64_t k,
                   const void* w, const void* x) {
    if (op == CQ_OP_INT4GEMV) return cq::plan_int4(v.kind, v.rows, n, k, w, x);
    if (op == CQ_OP_QGEMV) return cq::plan_q8(v.kind, v.rows, n, k, w, x);
    return cq::plan_gemv(v.kind, gemv_dtype(op), n, k, w, x);
}

hipError_t launch_plan(int op, const cq::Plan& p, const void* w,
                       const void* scale, const void* x, void* y, int64_t n,
                       int64_t k, hipStream_t stream, hipEvent_t ev0,
                       hipEvent_t ev1) {
    if (op == CQ_OP_INT4GEMV)
        return cq::launch_int4(p, w, scale, x, y, n, k, stream, ev0, ev1);
    if (op == CQ_OP_QGEMV)
        return cq::launch_q8(p, w, scale, x, y, n, k, stream, ev0, ev1);
    return cq::launch_gemv(p, gemv_dtype(op), w, x, y, n, k, stream, ev0, ev1);
}

hipError_t prepare_plan(int op, const cq::Plan& p, const void* w,
                        const void* scale, const void* x, void* y, int64_t n,
                        int64_t k, cq::Launch* out) {
    if (op == CQ_OP_INT4GEMV) return cq::prepare_int4(p, w, scale, x, y, n, k, out);
    if (op == CQ_OP_QGEMV) return cq::prepare_q8(p, w, scale, x, y, n, k, out);
    return cq::prepare_gemv(p, gemv_dtype(op), w, x, y, n, k, out);
}

// Layout of a filled cq_prepared_t: a magic word, a seal over the launch
// record (FNV-1a of its bytes, keyed by the magic) and the record itself.
struct Prepared {
    uint64_t magic;
    uint64_t seal;
    cq::Launch launch;
};
static_assert(sizeof(Prepared) <= sizeof(cq_prepared_t), "cq_prepared_t too small");
static_assert(std::is_trivially_copyable_v<cq::Launch>);
constexpr uint64_t kPreparedMagic = 0x31766d6771616463ull;  // "cdaqgmv1"

uint64_t seal_of(const cq::Launch& L) {
    unsigned char bytes[sizeof(cq::Launch)];
    std::memcpy(bytes, &L, sizeof bytes);
    uint64_t h = 0xcbf29ce484222325ull ^ kPreparedMagic;
    for (unsigned char b : bytes) h = (h ^ b) * 0x100000001b3ull;
    return h;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(CQ_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) +
                                " (" + hipGetErrorString(e) + ")");
}

int run_one(int op, const char* variant, const void* w, const void* scale,
            const void* x, void* y, int64_t n, int64_t k, void* stream) {
    g_last_error.clear();
    const Variant* v = nullptr;
    const int st = check_launch(op, variant, &v, w, scale, x, y, n, k);
    if (st != CQ_OK) return st;
    const cq::Plan p = make_plan(op, *v, n, k, w, x);
    const hipError_t e = launch_plan(op, p, w, scale, x, y, n, k,
                                     static_cast<hipStream_t>(stream), nullptr, nullptr);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return CQ_OK;
}

// Argument checks of the quantizer entry points (plain pointers and sizes;
// the Python layer keeps the reference's ValueError checks on metadata).
int check_quantize(int op, const void* w, const void* q, const void* scale,
                   int64_t n, int64_t k, int scale_mode) {
    if (scale_mode != CQ_SCALE_DIV && scale_mode != CQ_SCALE_RCP)
        return fail(CQ_ERR_INVALID_ARG, "unknown scale_mode " + std::to_string(scale_mode));
    if (w == nullptr || q == nullptr || scale == nullptr)
        return fail(CQ_ERR_INVALID_ARG, "null pointer argument");
    if (n < 1 || k < 1 || n > INT_MAX || k > INT_MAX)
        return fail(CQ_ERR_INVALID_ARG, "n and k must be in [1, INT_MAX] (n=" +
                                            std::to_string(n) + ", k=" + std::to_string(k) + ")");
    if (op == CQ_OP_INT4GEMV && k % 128 != 0)
        return fail(CQ_ERR_INVALID_ARG, "k must be divisible by 128 (got k=" +
                                            std::to_string(k) + ")");
    const uintptr_t sa = op == CQ_OP_INT4GEMV ? 2 : 4;
    if ((reinterpret_cast<uintptr_t>(w) & 1u) != 0 ||
        reinterpret_cast<uintptr_t>(scale) % sa != 0)
        return fail(CQ_ERR_INVALID_ARG, "w must be 2-byte aligned and scale aligned "
                                        "to its element size");
    // The kernels read w while other workgroups write the packed weights
    // and scales: the three ranges must be disjoint.  operand_spans gives
    // the packed weights' and scales' ranges for the operator (as "w" and
    // "scale"); the fp16 input is n * k * 2 bytes.
    const Operands o = operand_spans(op, q, scale, nullptr, nullptr, n, k);
    Span in;
    in.lo = reinterpret_cast<uintptr_t>(w);
    in.hi = in.lo + static_cast<unsigned __int128>(n) * static_cast<unsigned __int128>(k) * 2;
    if (overlaps(in, o.w) || overlaps(in, o.scale) || overlaps(o.w, o.scale))
        return fail(CQ_ERR_INVALID_ARG, "w, the quantized output and scale must not "
                                        "overlap");
    return CQ_OK;
}

int run_grouped(int op, const char* variant, const cq_gemv_problem_t* probs,
                int64_t count, int64_t k, void* stream) {
    g_last_error.clear();
    if (probs == nullptr) return fail(CQ_ERR_INVALID_ARG, "problems is NULL");
    if (count < 1 || count > INT_MAX)
        return fail(CQ_ERR_INVALID_ARG, "n_problems must be >= 1, got " + std::to_string(count));
    const Variant* v = nullptr;
    for (int64_t i = 0; i < count; ++i) {
        const cq_gemv_problem_t& q = probs[i];
        const int st = check_launch(op, variant, &v, q.w, q.scale, q.x, q.y, q.n, k);
        if (st != CQ_OK) {
            g_last_error = "problem " + std::to_string(i) + ": " + g_last_error;
            return st;
        }
    }
    // Problems of one launch run concurrently: no output may share a byte
    // with another problem's operands or output (inputs may be shared, as
    // q/k/v share x).  The outputs are sorted by address: adjacent ones
    // must not overlap, and then each input span is looked up among them.
    std::vector<Operands> ops(static_cast<size_t>(count));
    std::vector<int64_t> by_y(static_cast<size_t>(count));
    for (int64_t i = 0; i < count; ++i) {
        const cq_gemv_problem_t& q = probs[i];
        ops[static_cast<size_t>(i)] = operand_spans(op, q.w, q.scale, q.x, q.y, q.n, k);
        by_y[static_cast<size_t>(i)] = i;
    }
    auto ys = [&](int64_t i) -> const Span& { return ops[static_cast<size_t>(i)].y; };
    std::sort(by_y.begin(), by_y.end(),
              [&](int64_t a, int64_t b) { return ys(a).lo < ys(b).lo; });
    auto conflict = [&](int64_t i, const char* what, int64_t j) {
        return fail(CQ_ERR_INVALID_ARG,
                    "problem " + std::to_string(i) + ": output y overlaps " + what +
                        " of problem " + std::to_string(j) +
                        " (the problems of a grouped call must be independent)");
    };
    for (size_t t = 1; t < by_y.size(); ++t)
        if (overlaps(ys(by_y[t - 1]), ys(by_y[t])))
            return conflict(by_y[t], "y", by_y[t - 1]);
    for (int64_t j = 0; j < count; ++j) {
        const Operands& o = ops[static_cast<size_t>(j)];
        const std::pair<const Span*, const char*> inputs[] = {
            {&o.w, "w"}, {&o.scale, "scale"}, {&o.x, "x"}};
        for (const auto& [sp, what] : inputs) {
            // first output ending after the input starts; outputs are
            // disjoint, so their ends are sorted too
            auto it = std::partition_point(by_y.begin(), by_y.end(), [&](int64_t i) {
                return ys(i).hi <= sp->lo;
            });
            for (; it != by_y.end() && ys(*it).lo < sp->hi; ++it)
                if (*it != j && overlaps(ys(*it), *sp)) return conflict(*it, what, j);
        }
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto one = [&](const cq_gemv_problem_t& q) {
        const cq::Plan p = make_plan(op, *v, q.n, k, q.w, q.x);
        return launch_plan(op, p, q.w, q.scale, q.x, q.y, q.n, k, s, nullptr, nullptr);
    };
    for (int64_t off = 0; off < count; off += cq::kMaxGroup) {
        const int c = static_cast<int>(std::min<int64_t>(cq::kMaxGroup, count - off));
        hipError_t e = hipSuccess;
        cq::Plan p;
        cq::GroupProblem gp[cq::kMaxGroup];
        for (int i = 0; i < c; ++i) {
            const cq_gemv_problem_t& q = probs[off + i];
            gp[i] = {q.w, q.scale, q.x, q.y, q.n};
        }
        if (v->kind == cq::kLds)
            p = op == CQ_OP_INT4GEMV ? cq::plan_int4_group(v->rows, gp, c, k)
                                     : cq::plan_q8_group(v->rows, gp, c, k);
        if (v->kind == cq::kLds && p.kind == cq::kLds) {
            e = op == CQ_OP_INT4GEMV ? cq::launch_int4_group(p, gp, c, k, s)
                                     : cq::launch_q8_group(p, gp, c, k, s);
        } else {
            for (int i = 0; i < c && e == hipSuccess; ++i) e = one(probs[off + i]);
        }
        if (e != hipSuccess) return hip_fail(e, "grouped launch");
    }
    return CQ_OK;
}

std::string join_sorted(std::vector<std::string> names) {
    std::sort(names.begin(), names.end());
    std::string s;
    for (size_t i = 0; i < names.size(); ++i) {
        if (i) s += '\n';
        s += names[i];
    }
    return s;
}

int write_out(const std::string& s, char* buf, size_t cap) {
    const size_t need = s.size() + 1;
    if (need > static_cast<size_t>(INT_MAX)) return fail(CQ_ERR_INVALID_ARG, "string too long");
    if (buf != nullptr && cap >= need) std::memcpy(buf, s.c_str(), need);
    return static_cast<int>(need);
}

// Event pair owned for the duration of a timing call.
struct Events {
    std::vector<hipEvent_t> ev;
    ~Events() {
        for (hipEvent_t e : ev)
            if (e != nullptr) (void)hipEventDestroy(e);
    }
    hipError_t make(size_t count) {
        ev.assign(count, nullptr);
        for (auto& e : ev) {
            const hipError_t r = hipEventCreate(&e);
            if (r != hipSuccess) return r;
        }
        return hipSuccess;
    }
};

// Options of the timing loops' window (see cq_pool_timing).
struct Window {
    int64_t warmup;     // untimed launches, at least
    double burn_ms;     // and at least this much wall-clock time of them
    double delay_us;    // > 0: on-device wait queued ahead of the window
    int64_t n_launches;
};

int check_window(const Window& w) {
    if (w.warmup < 0) return fail(CQ_ERR_INVALID_ARG, "warmup must be >= 0");
    if (w.n_launches < 1) return fail(CQ_ERR_INVALID_ARG, "n_launches must be >= 1");
    if (!std::isfinite(w.burn_ms) || w.burn_ms < 0 || w.burn_ms > 600000)
        return fail(CQ_ERR_INVALID_ARG, "burn_ms must be in [0, 600000]");
    if (!std::isfinite(w.delay_us) || w.delay_us < 0 || w.delay_us > 1e6)
        return fail(CQ_ERR_INVALID_ARG, "delay_us must be in [0, 1e6]");
    return CQ_OK;
}

// The shared timing loop.  `go(i, ev0, ev1)` enqueues launch i (ev0/ev1
// non-null: events on the dispatch itself).  Untimed launches run until
// both `warmup` launches and `burn_ms` of wall-clock time have passed
// (clocks and power settle); the stream is synchronized; a delay of
// `delay_us` is queued; then the start event, the n_launches timed
// launches and the stop event.  *total_us is the event time of the window,
// *host_us (if non-null) the host time spent enqueuing it: a window whose
// host time reaches its event time was bound by submission, not the GPU.
template <typename Go>
int timed_window(Go go, hipStream_t s, const Window& w, float* kernel_us,
                 double* total_us, double* host_us) {
    using clock = std::chrono::steady_clock;
    hipError_t e;
    const auto t_burn = clock::now();
    int64_t i = 0;
    while (i < w.warmup ||
           std::chrono::duration<double, std::milli>(clock::now() - t_burn).count() < w.burn_ms) {
        if ((e = go(i, nullptr, nullptr)) != hipSuccess) return hip_fail(e, "warmup launch");
        ++i;
    }
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    Events win;
    if ((e = win.make(2)) != hipSuccess) return hip_fail(e, "hipEventCreate");
    Events per;
    if (kernel_us != nullptr &&
        (e = per.make(2 * static_cast<size_t>(w.n_launches))) != hipSuccess)
        return hip_fail(e, "hipEventCreate");
    if ((e = cq::launch_delay(w.delay_us, s)) != hipSuccess) return hip_fail(e, "delay launch");
    if ((e = hipEventRecord(win.ev[0], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
    const auto t_enq = clock::now();
    for (int64_t j = 0; j < w.n_launches; ++j) {
        hipEvent_t e0 = kernel_us ? per.ev[2 * static_cast<size_t>(j)] : nullptr;
        hipEvent_t e1 = kernel_us ? per.ev[2 * static_cast<size_t>(j) + 1] : nullptr;
        if ((e = go(i + j, e0, e1)) != hipSuccess) return hip_fail(e, "timed launch");
    }
    const double enq_us = std::chrono::duration<double, std::micro>(clock::now() - t_enq).count();
    if ((e = hipEventRecord(win.ev[1], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
    if ((e = hipEventSynchronize(win.ev[1])) != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    float ms = 0.f;
    if ((e = hipEventElapsedTime(&ms, win.ev[0], win.ev[1])) != hipSuccess)
        return hip_fail(e, "hipEventElapsedTime");
    if (total_us != nullptr) *total_us = static_cast<double>(ms) * 1e3;
    if (host_us != nullptr) *host_us = enq_us;
    if (kernel_us != nullptr) {
        for (int64_t j = 0; j < w.n_launches; ++j) {
            float kms = 0.f;
            e = hipEventElapsedTime(&kms, per.ev[2 * static_cast<size_t>(j)],
                                    per.ev[2 * static_cast<size_t>(j) + 1]);
            if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime (kernel)");
            kernel_us[j] = kms * 1e3f;
        }
    }
    return CQ_OK;
}

}  // namespace

extern "C" {

int cq_int4gemv(const char* variant, const void* w_packed, const void* scale,
                const void* x, void* y, int64_t n, int64_t k, void* stream) {
    return run_one(CQ_OP_INT4GEMV, variant, w_packed, scale, x, y, n, k, stream);
}

int cq_qgemv(const char* variant, const void* w_q, const void* scale,
             const void* x, void* y, int64_t n, int64_t k, void* stream) {
    return run_one(CQ_OP_QGEMV, variant, w_q, scale, x, y, n, k, stream);
}

int cq_gemv(const char* variant, int dtype, const void* w, const void* x,
            void* y, int64_t n, int64_t k, void* stream) {
    if (dtype != CQ_DTYPE_F16 && dtype != CQ_DTYPE_F32) {
        g_last_error = "unknown gemv dtype " + std::to_string(dtype);
        return CQ_ERR_INVALID_ARG;
    }
    return run_one(dtype == CQ_DTYPE_F32 ? CQ_OP_GEMV_F32 : CQ_OP_GEMV_F16,
                   variant, w, nullptr, x, y, n, k, stream);
}

int cq_int4gemv_grouped(const char* variant, const cq_gemv_problem_t* problems,
                        int64_t n_problems, int64_t k, void* stream) {
    return run_grouped(CQ_OP_INT4GEMV, variant, problems, n_problems, k, stream);
}

int cq_qgemv_grouped(const char* variant, const cq_gemv_problem_t* problems,
                     int64_t n_problems, int64_t k, void* stream) {
    return run_grouped(CQ_OP_QGEMV, variant, problems, n_problems, k, stream);
}

int cq_int4_quantize(const void* w, void* w_packed, void* scale, int64_t n,
                     int64_t k, int scale_mode, void* stream) {
    g_last_error.clear();
    int st = check_quantize(CQ_OP_INT4GEMV, w, w_packed, scale, n, k, scale_mode);
    if (st != CQ_OK) return st;
    const cq::QuantPlan p = cq::plan_int4_quantize(n, k, w, w_packed);
    if (p.grid > INT_MAX) return fail(CQ_ERR_INVALID_ARG, "n * k too large for one launch");
    const hipError_t e = cq::launch_int4_quantize(p, w, w_packed, scale, n, k,
                                                  scale_mode == CQ_SCALE_RCP,
                                                  static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return CQ_OK;
}

int cq_q8_quantize(const void* w, void* w_q, void* scale, int64_t n, int64_t k,
                   int scale_mode, void* stream) {
    g_last_error.clear();
    int st = check_quantize(CQ_OP_QGEMV, w, w_q, scale, n, k, scale_mode);
    if (st != CQ_OK) return st;
    const cq::QuantPlan p = cq::plan_q8_quantize(n, k, w, w_q);
    const hipError_t e = cq::launch_q8_quantize(p, w, w_q, scale, n, k,
                                                scale_mode == CQ_SCALE_RCP,
                                                static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return CQ_OK;
}

int cq_quantize_vectorized(int op, const void* w, const void* out, int64_t n,
                           int64_t k) {
    if (op == CQ_OP_INT4GEMV) return cq::plan_int4_quantize(n, k, w, out).fast ? 1 : 0;
    if (op == CQ_OP_QGEMV) return cq::plan_q8_quantize(n, k, w, out).fast ? 1 : 0;
    fail(CQ_ERR_INVALID_ARG, "quantizers exist for CQ_OP_INT4GEMV and CQ_OP_QGEMV only");
    return -1;
}

int cq_native_timing(int op, const char* variant, const void* w,
                     const void* scale, const void* x, void* y, int64_t n,
                     int64_t k, void* stream, int64_t warmup,
                     int64_t n_windows, int64_t launches_per_window,
                     double* window_us, cq_timing_t* out) {
    g_last_error.clear();
    if (warmup < 0) return fail(CQ_ERR_INVALID_ARG, "warmup must be >= 0");
    if (n_windows < 1) return fail(CQ_ERR_INVALID_ARG, "n_windows must be >= 1");
    if (launches_per_window < 1)
        return fail(CQ_ERR_INVALID_ARG, "launches_per_window must be >= 1");
    const Variant* v = nullptr;
    int st = check_launch(op, variant, &v, w, scale, x, y, n, k);
    if (st != CQ_OK) return st;
    const cq::Plan p = make_plan(op, *v, n, k, w, x);
    hipStream_t s = static_cast<hipStream_t>(stream);

    for (int64_t i = 0; i < warmup; ++i) {
        const hipError_t e = launch_plan(op, p, w, scale, x, y, n, k, s, nullptr, nullptr);
        if (e != hipSuccess) return hip_fail(e, "warmup launch");
    }
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");

    Events evs;
    if ((e = evs.make(2)) != hipSuccess) return hip_fail(e, "hipEventCreate");
    std::vector<double> per(static_cast<size_t>(n_windows));
    for (int64_t wdx = 0; wdx < n_windows; ++wdx) {
        if ((e = hipEventRecord(evs.ev[0], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
        for (int64_t i = 0; i < launches_per_window; ++i) {
            e = launch_plan(op, p, w, scale, x, y, n, k, s, nullptr, nullptr);
            if (e != hipSuccess) return hip_fail(e, "timed launch");
        }
        if ((e = hipEventRecord(evs.ev[1], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
        if ((e = hipEventSynchronize(evs.ev[1])) != hipSuccess) return hip_fail(e, "hipEventSynchronize");
        float ms = 0.f;
        if ((e = hipEventElapsedTime(&ms, evs.ev[0], evs.ev[1])) != hipSuccess)
            return hip_fail(e, "hipEventElapsedTime");
        per[static_cast<size_t>(wdx)] =
            static_cast<double>(ms) * 1e3 / static_cast<double>(launches_per_window);
    }
    if (window_us != nullptr) std::copy(per.begin(), per.end(), window_us);
    if (out != nullptr) {
        std::vector<double> srt = per;
        std::sort(srt.begin(), srt.end());
        const size_t m = srt.size();
        out->warmup = warmup;
        out->n_windows = n_windows;
        out->launches_per_window = launches_per_window;
        out->median_us = (m % 2 == 1) ? srt[m / 2] : 0.5 * (srt[m / 2 - 1] + srt[m / 2]);
        out->min_us = srt.front();
        out->max_us = srt.back();
        out->mean_us = std::accumulate(srt.begin(), srt.end(), 0.0) / static_cast<double>(m);
    }
    return CQ_OK;
}

int cq_pool_timing(int op, const char* variant, const void* const* w,
                   const void* const* scale, const void* const* x,
                   void* const* y, int64_t n_sets, int64_t n, int64_t k,
                   void* stream, int64_t warmup, double burn_ms,
                   double delay_us, int64_t n_launches, float* kernel_us,
                   double* total_us, double* host_us) {
    g_last_error.clear();
    if (w == nullptr || (scale == nullptr && !is_gemv(op)) || x == nullptr ||
        y == nullptr)
        return fail(CQ_ERR_INVALID_ARG, "null set array");
    if (n_sets < 1) return fail(CQ_ERR_INVALID_ARG, "n_sets must be >= 1");
    const Window win{warmup, burn_ms, delay_us, n_launches};
    int st = check_window(win);
    if (st != CQ_OK) return st;
    std::vector<cq::Plan> plans(static_cast<size_t>(n_sets));
    const Variant* v = nullptr;
    for (int64_t i = 0; i < n_sets; ++i) {
        const void* sc = scale != nullptr ? scale[i] : nullptr;
        st = check_launch(op, variant, &v, w[i], sc, x[i], y[i], n, k);
        if (st != CQ_OK) return st;
        plans[static_cast<size_t>(i)] = make_plan(op, *v, n, k, w[i], x[i]);
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](int64_t i, hipEvent_t e0, hipEvent_t e1) {
        const size_t si = static_cast<size_t>(i % n_sets);
        return launch_plan(op, plans[si], w[si], scale != nullptr ? scale[si] : nullptr,
                           x[si], y[si], n, k, s, e0, e1);
    };
    return timed_window(go, s, win, kernel_us, total_us, host_us);
}

int cq_read_ceiling(const void* const* bufs, int64_t n_bufs, int64_t bytes,
                    void* sink, void* stream, int64_t warmup, double burn_ms,
                    double delay_us, int64_t n_launches, double* total_us) {
    g_last_error.clear();
    if (bufs == nullptr || sink == nullptr || total_us == nullptr)
        return fail(CQ_ERR_INVALID_ARG, "null argument");
    if (n_bufs < 1) return fail(CQ_ERR_INVALID_ARG, "n_bufs must be >= 1");
    const Window win{warmup, burn_ms, delay_us, n_launches};
    const int st = check_window(win);
    if (st != CQ_OK) return st;
    if (bytes < 16 || bytes % 16 != 0)
        return fail(CQ_ERR_INVALID_ARG, "bytes must be a positive multiple of 16");
    for (int64_t i = 0; i < n_bufs; ++i)
        if (bufs[i] == nullptr || (reinterpret_cast<uintptr_t>(bufs[i]) & 15u) != 0)
            return fail(CQ_ERR_INVALID_ARG, "buffers must be non-null and 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](int64_t i, hipEvent_t, hipEvent_t) {
        return cq::launch_stream_read(bufs[i % n_bufs], bytes, sink, s);
    };
    return timed_window(go, s, win, nullptr, total_us, nullptr);
}

int cq_launch_floor(int64_t grid, int block, void* sink, void* stream,
                    int64_t warmup, double burn_ms, double delay_us,
                    int64_t n_launches, double* total_us) {
    g_last_error.clear();
    if (sink == nullptr || total_us == nullptr)
        return fail(CQ_ERR_INVALID_ARG, "null argument");
    const Window win{warmup, burn_ms, delay_us, n_launches};
    const int st = check_window(win);
    if (st != CQ_OK) return st;
    if (grid < 1 || grid > INT_MAX || block < 1 || block > 1024)
        return fail(CQ_ERR_INVALID_ARG,
                    "grid must be in [1, INT_MAX] and block in [1, 1024]");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](int64_t, hipEvent_t, hipEvent_t) {
        return cq::launch_empty(grid, block, sink, s);
    };
    return timed_window(go, s, win, nullptr, total_us, nullptr);
}

int cq_int4_timeline(const char* variant, const void* const* w,
                     const void* const* scale, const void* const* x,
                     void* const* y, int64_t n_sets, int64_t n, int64_t k,
                     void* stream, int64_t warmup, double burn_ms,
                     double delay_us, int64_t n_launches, uint64_t* stamps,
                     int64_t stamps_words, int64_t* waves_out,
                     double* ticks_per_us, double* total_us) {
    g_last_error.clear();
    if (w == nullptr || scale == nullptr || x == nullptr || y == nullptr ||
        stamps == nullptr || waves_out == nullptr || ticks_per_us == nullptr ||
        total_us == nullptr)
        return fail(CQ_ERR_INVALID_ARG, "null argument");
    if (n_sets < 1) return fail(CQ_ERR_INVALID_ARG, "n_sets must be >= 1");
    const Window win{warmup, burn_ms, delay_us, n_launches};
    int st = check_window(win);
    if (st != CQ_OK) return st;
    std::vector<cq::Plan> plans(static_cast<size_t>(n_sets));
    const Variant* v = nullptr;
    for (int64_t i = 0; i < n_sets; ++i) {
        st = check_launch(CQ_OP_INT4GEMV, variant, &v, w[i], scale[i], x[i], y[i], n, k);
        if (st != CQ_OK) return st;
        cq::Plan& p = plans[static_cast<size_t>(i)];
        p = make_plan(CQ_OP_INT4GEMV, *v, n, k, w[i], x[i]);
        if (p.kind != cq::kLds)
            return fail(CQ_ERR_INVALID_ARG,
                        std::string("the timeline covers the LDS kernel; ") + v->name +
                            " plans another kernel for set " + std::to_string(i));
        if (p.grid != plans[0].grid || p.block != plans[0].block)
            return fail(CQ_ERR_INVALID_ARG, "the sets' plans differ in launch shape");
    }
    const int64_t waves = plans[0].grid * (plans[0].block / 64);
    if (n_launches > (INT64_MAX / 8) / waves || stamps_words < n_launches * waves * 8)
        return fail(CQ_ERR_INVALID_ARG,
                    "stamps holds " + std::to_string(stamps_words) + " words; " +
                        std::to_string(n_launches) + " launches of " +
                        std::to_string(waves) + " waves need 8 per wave");
    // the kernel writes the stamps while it reads the sets: no shared byte
    Span sp;
    sp.lo = reinterpret_cast<uintptr_t>(stamps);
    sp.hi = sp.lo + static_cast<unsigned __int128>(n_launches * waves * 8) * 8;
    for (int64_t i = 0; i < n_sets; ++i) {
        const Operands o = operand_spans(CQ_OP_INT4GEMV, w[i], scale[i], x[i], y[i], n, k);
        if (overlaps(sp, o.w) || overlaps(sp, o.scale) || overlaps(sp, o.x) ||
            overlaps(sp, o.y))
            return fail(CQ_ERR_INVALID_ARG,
                        "stamps overlap an operand of set " + std::to_string(i));
    }
    int dev = 0, khz = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    if (khz <= 0) return fail(CQ_ERR_HIP, "the device reports no wall clock rate");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](int64_t i, hipEvent_t, hipEvent_t) {
        const size_t si = static_cast<size_t>(i % n_sets);
        uint64_t* slot = stamps + (i % n_launches) * waves * 8;
        return cq::launch_int4_stamped(plans[si], w[si], scale[si], x[si], y[si], n, k,
                                       slot, s);
    };
    st = timed_window(go, s, win, nullptr, total_us, nullptr);
    if (st != CQ_OK) return st;
    *waves_out = waves;
    *ticks_per_us = static_cast<double>(khz) / 1000.0;
    return CQ_OK;
}

int cq_variants(int op, int which, char* buf, size_t cap) {
    g_last_error.clear();
    if (!valid_op(op))
        return fail(-CQ_ERR_INVALID_ARG, "unknown operator id " + std::to_string(op));
    op = family(op);
    std::vector<std::string> names;
    if (which == CQ_LIST_ALIASES) {
        for (const Alias& a : kAliases)
            if (a.op == op) names.push_back(std::string(a.alias) + "=" + a.target);
    } else if (which == CQ_LIST_NORMAL || which == CQ_LIST_ALL ||
               which == CQ_LIST_QUARANTINED) {
        for (const Variant& v : kVariants) {
            if (v.op != op) continue;
            if (which == CQ_LIST_NORMAL && v.quarantined) continue;
            if (which == CQ_LIST_QUARANTINED && !v.quarantined) continue;
            names.push_back(v.name);
        }
    } else {
        return fail(-CQ_ERR_INVALID_ARG, "unknown list selector " + std::to_string(which));
    }
    return write_out(join_sorted(names), buf, cap);
}

int cq_vec_contract_ok(int op, const void* w, const void* x, int64_t k) {
    if (op == CQ_OP_INT4GEMV) return cq::int4_contract_ok(w, x, k) ? 1 : 0;
    if (op == CQ_OP_QGEMV) return cq::q8_contract_ok(w, x, k) ? 1 : 0;
    if (is_gemv(op)) return cq::gemv_contract_ok(gemv_dtype(op), w, x, k) ? 1 : 0;
    return 0;
}

int cq_describe_launch(int op, const char* variant, int64_t n, int64_t k,
                       const void* w, const void* x, char* buf, size_t cap) {
    g_last_error.clear();
    const Variant* v = nullptr;
    // describe with stand-in scale/y pointers: only w/x alignment matters
    const int st = check_call(op, variant, &v, w, w, x, w, n, k);
    if (st != CQ_OK) return -st;
    const cq::Plan p = make_plan(op, *v, n, k, w, x);
    // the launch the plan resolves to (nothing is enqueued), for its LDS bytes
    cq::Launch L;
    const void* sc = is_gemv(op) ? nullptr : w;
    const long long lds = prepare_plan(op, p, w, sc, x, const_cast<void*>(w), n, k, &L) == hipSuccess
                              ? static_cast<long long>(L.shmem) : -1;
    char line[512];
    std::snprintf(line, sizeof line,
                  "variant=%s kernel=%s cw=%d j=%d r=%d tile=%d block=%d grid=%lld lds=%lld fallback=%d why=%s",
                  v->name,
                  p.kind == cq::kScalar ? "scalar"
                  : p.kind == cq::kLds  ? "lds"
                  : p.kind == cq::kTiled ? "tiled"
                                         : "wave",
                  p.cw, p.j, p.r, p.tile,
                  p.block, static_cast<long long>(p.grid), lds, p.fallback ? 1 : 0,
                  p.why.empty() ? "-" : p.why.c_str());
    return write_out(line, buf, cap);
}

int cq_prepare(int op, const char* variant, const void* w, const void* scale,
               const void* x, void* y, int64_t n, int64_t k, cq_prepared_t* out) {
    g_last_error.clear();
    if (out == nullptr) return fail(CQ_ERR_INVALID_ARG, "prepared record pointer is NULL");
    std::memset(out, 0, sizeof *out);
    if (is_gemv(op)) scale = nullptr;
    const Variant* v = nullptr;
    const int st = check_launch(op, variant, &v, w, scale, x, y, n, k);
    if (st != CQ_OK) return st;
    const cq::Plan p = make_plan(op, *v, n, k, w, x);
    Prepared rec{};
    const hipError_t e = prepare_plan(op, p, w, scale, x, y, n, k, &rec.launch);
    if (e != hipSuccess) return hip_fail(e, "launch preparation");
    rec.magic = kPreparedMagic;
    rec.seal = seal_of(rec.launch);
    std::memcpy(out, &rec, sizeof rec);
    return CQ_OK;
}

int cq_launch_prepared(const cq_prepared_t* prepared, void* stream) {
    g_last_error.clear();
    if (prepared == nullptr) return fail(CQ_ERR_INVALID_ARG, "prepared record pointer is NULL");
    Prepared rec;
    std::memcpy(&rec, prepared, sizeof rec);
    if (rec.magic != kPreparedMagic || rec.seal != seal_of(rec.launch))
        return fail(CQ_ERR_INVALID_ARG, "not a record filled by cq_prepare (or damaged)");
    const hipError_t e = cq::enqueue(rec.launch, static_cast<hipStream_t>(stream),
                                     nullptr, nullptr);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return CQ_OK;
}

const char* cq_last_error(void) { return g_last_error.c_str(); }

// The build passes CQ_SRC_HASH, a stamp of the sources and flags the
// library was compiled from; the Python loader compares it with the tree.
#ifndef CQ_SRC_HASH
#define CQ_SRC_HASH "unstamped"
#endif
const char* cq_version(void) { return "cdnaqgemv 0.2.0 (gfx950) src=" CQ_SRC_HASH; }

}  // extern "C"
