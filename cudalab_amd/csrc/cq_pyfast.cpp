// Fast path of the eager Python API (cudalab_amd/ext.py): one call from
// Python checks the tensors of a forward / forward_into call on their
// metadata, finds the launch in a cache of prepared launches (cq_prepare,
// keyed by variant, operand addresses and sizes) and enqueues it on the
// current HIP stream of the operands' device (cq_launch_prepared).  Grouped
// calls (forward_grouped) take the same checks per problem and go to the
// library's grouped entry point directly.
//
// The reference's bindings do their checks and the launch in C++ as well
// (kernels/int4gemv/bindings.cpp:60-176, kernels/qgemv/bindings.cpp:65-173,
// kernels/gemv/bindings.cpp:87-190).  Here the Python layer keeps the
// checks that raise, in the reference's order and with its messages; this
// file decides no error.  Every function returns "not taken" (false /
// None), launching nothing, unless all of the following hold, and the
// Python layer then runs its checked path:
//   * the variant is a name the operator accepts (registered or alias);
//   * every operand is a torch tensor, strided, contiguous, of the
//     operator's dtype and shape, and on one GPU, the current device;
//   * cq_prepare accepts the call (it refuses, e.g., an output overlapping
//     an input).
// A launch error after all of that raises RuntimeError with the message the
// checked path would give ("<op> launch failed (status N): <error>").
//
// The library's entry points are bound by address (taken from the ctypes
// handle of libcdnaqgemv.so), so this module and the ctypes layer share one
// loaded library and one per-thread error string.
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/python_variable.h>
#include <torch/csrc/utils/pybind.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "cdnaqgemv.h"

namespace py = pybind11;

#ifndef CQ_FAST_ABI
#define CQ_FAST_ABI "unstamped"
#endif
#ifndef CQ_SRC_HASH
#define CQ_SRC_HASH "unstamped"
#endif

namespace {

using PrepareFn = int (*)(int, const char*, const void*, const void*, const void*,
                          void*, int64_t, int64_t, cq_prepared_t*);
using LaunchFn = int (*)(const cq_prepared_t*, void*);
using ErrorFn = const char* (*)();
using GroupedFn = int (*)(const char*, const cq_gemv_problem_t*, int64_t, int64_t, void*);

enum Kind { kInt4 = 0, kQ8 = 1, kGemv = 2 };

struct Key {
    const void* w;
    const void* s;
    const void* x;
    const void* y;
    int64_t n;
    int64_t k;
    int32_t variant;
    int32_t op;
    bool operator==(const Key& o) const {
        return w == o.w && s == o.s && x == o.x && y == o.y && n == o.n &&
               k == o.k && variant == o.variant && op == o.op;
    }
};

struct KeyHash {
    size_t operator()(const Key& k) const noexcept {
        uint64_t h = 0x9e3779b97f4a7c15ull;
        auto mix = [&h](uint64_t v) {
            h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
        };
        mix(reinterpret_cast<uintptr_t>(k.w));
        mix(reinterpret_cast<uintptr_t>(k.s));
        mix(reinterpret_cast<uintptr_t>(k.x));
        mix(reinterpret_cast<uintptr_t>(k.y));
        mix(static_cast<uint64_t>(k.n));
        mix(static_cast<uint64_t>(k.k));
        mix((static_cast<uint64_t>(k.variant) << 8) | static_cast<uint64_t>(k.op));
        return static_cast<size_t>(h);
    }
};

bool plain(const at::Tensor& t, at::ScalarType dtype) {
    return t.defined() && t.layout() == at::kStrided && t.scalar_type() == dtype &&
           t.is_contiguous();
}

// Device rule shared by every operand: the first operand's device, which
// must be a GPU and the current device when `require_gpu` (tests run the
// metadata rule on CPU tensors with require_gpu = false).
bool same_device(const at::Tensor& w, std::initializer_list<const at::Tensor*> rest,
                 bool require_gpu) {
    const c10::Device d = w.device();
    for (const at::Tensor* t : rest)
        if (t->device() != d) return false;
    if (!require_gpu) return true;
    return d.is_cuda() && d.index() == c10::hip::current_device();
}

class Launcher {
public:
    Launcher(int kind, const std::vector<std::string>& names, uintptr_t prepare,
             uintptr_t launch, uintptr_t last_error, int64_t capacity,
             uintptr_t grouped)
        : kind_(kind),
          prepare_(reinterpret_cast<PrepareFn>(prepare)),
          launch_(reinterpret_cast<LaunchFn>(launch)),
          last_error_(reinterpret_cast<ErrorFn>(last_error)),
          grouped_(reinterpret_cast<GroupedFn>(grouped)),
          capacity_(capacity < 1 ? 1 : static_cast<size_t>(capacity)),
          names_(names) {
        if (kind < kInt4 || kind > kGemv) throw std::invalid_argument("unknown operator kind");
        if (prepare_ == nullptr || launch_ == nullptr || last_error_ == nullptr)
            throw std::invalid_argument("null library entry point");
        for (size_t i = 0; i < names_.size(); ++i)
            ids_.emplace(std::string_view(names_[i]), static_cast<int32_t>(i));
    }
    // ids_ views the strings of names_: a copy would view the original's
    Launcher(const Launcher&) = delete;
    Launcher& operator=(const Launcher&) = delete;

    // ---- the metadata rule, for tests (no launch, no cache) ----
    bool accepts(const at::Tensor& w, const at::Tensor& scale, const at::Tensor& x,
                 const at::Tensor& out, bool require_gpu) const {
        return kind_ != kGemv && quant_ok(w, scale, x, &out, require_gpu);
    }
    bool gemv_accepts(const at::Tensor& w, const at::Tensor& x, const at::Tensor& out,
                      bool require_gpu) const {
        return kind_ == kGemv && gemv_ok(w, x, &out, require_gpu);
    }

    // ---- INT4 / INT8: forward_into and forward ----
    // Operands arrive as plain Python objects so that a non-tensor argument
    // is "not taken" here (the checked path raises its own message) rather
    // than a binding TypeError.
    bool into(py::handle variant, py::handle w, py::handle scale, py::handle x,
              py::handle out) {
        const int32_t vid = variant_id(variant);
        if (vid < 0 || kind_ == kGemv || !all_tensors({w, scale, x, out})) return false;
        const at::Tensor& W = THPVariable_Unpack(w.ptr());
        const at::Tensor& S = THPVariable_Unpack(scale.ptr());
        const at::Tensor& X = THPVariable_Unpack(x.ptr());
        const at::Tensor& Y = THPVariable_Unpack(out.ptr());
        if (!quant_ok(W, S, X, &Y, true)) return false;
        return run(vid, W, S.data_ptr(), X, Y);
    }
    py::object forward(py::handle variant, py::handle w, py::handle scale, py::handle x) {
        const int32_t vid = variant_id(variant);
        if (vid < 0 || kind_ == kGemv || !all_tensors({w, scale, x})) return py::none();
        const at::Tensor& W = THPVariable_Unpack(w.ptr());
        const at::Tensor& S = THPVariable_Unpack(scale.ptr());
        const at::Tensor& X = THPVariable_Unpack(x.ptr());
        if (!quant_ok(W, S, X, nullptr, true)) return py::none();
        at::Tensor Y = at::empty({W.size(0)}, W.options().dtype(at::kHalf));
        if (!run(vid, W, S.data_ptr(), X, Y)) return py::none();
        return py::cast(Y);
    }

    // ---- FP16 / FP32 GEMV ----
    bool gemv_into(py::handle variant, py::handle w, py::handle x, py::handle out) {
        const int32_t vid = variant_id(variant);
        if (vid < 0 || kind_ != kGemv || !all_tensors({w, x, out})) return false;
        const at::Tensor& W = THPVariable_Unpack(w.ptr());
        const at::Tensor& X = THPVariable_Unpack(x.ptr());
        const at::Tensor& Y = THPVariable_Unpack(out.ptr());
        if (!gemv_ok(W, X, &Y, true)) return false;
        return run(vid, W, nullptr, X, Y);
    }
    py::object gemv_forward(py::handle variant, py::handle w, py::handle x) {
        const int32_t vid = variant_id(variant);
        if (vid < 0 || kind_ != kGemv || !all_tensors({w, x})) return py::none();
        const at::Tensor& W = THPVariable_Unpack(w.ptr());
        const at::Tensor& X = THPVariable_Unpack(x.ptr());
        if (!gemv_ok(W, X, nullptr, true)) return py::none();
        at::Tensor Y = at::empty({W.size(0)}, W.options());
        if (!run(vid, W, nullptr, X, Y)) return py::none();
        return py::cast(Y);
    }

    // ---- INT4 / INT8 grouped calls ----
    // `problems` must be a list or tuple (any other iterable is left
    // unconsumed for the checked path) of 4-item lists or tuples of
    // tensors, each accepted by the forward_into rule, all with one K and
    // on one device.  The library's grouped entry point then runs its own
    // checks (overlaps included); a refusal there is "not taken" too, so
    // the checked path raises it with the reference-style message.
    bool grouped(py::handle variant, py::handle problems) {
        const int32_t vid = variant_id(variant);
        if (vid < 0 || kind_ == kGemv || grouped_ == nullptr) return false;
        PyObject* seq = problems.ptr();
        if (!PyList_Check(seq) && !PyTuple_Check(seq)) return false;
        const Py_ssize_t count = PySequence_Fast_GET_SIZE(seq);
        if (count < 1) return false;
        std::vector<cq_gemv_problem_t> probs(static_cast<size_t>(count));
        int64_t k0 = 0;
        c10::Device dev0(c10::DeviceType::CPU);
        for (Py_ssize_t i = 0; i < count; ++i) {
            PyObject* item = PySequence_Fast_GET_ITEM(seq, i);
            if ((!PyTuple_Check(item) && !PyList_Check(item)) ||
                PySequence_Fast_GET_SIZE(item) != 4)
                return false;
            PyObject** f = PySequence_Fast_ITEMS(item);
            for (int j = 0; j < 4; ++j)
                if (!THPVariable_Check(f[j])) return false;
            const at::Tensor& W = THPVariable_Unpack(f[0]);
            const at::Tensor& S = THPVariable_Unpack(f[1]);
            const at::Tensor& X = THPVariable_Unpack(f[2]);
            const at::Tensor& Y = THPVariable_Unpack(f[3]);
            if (!quant_ok(W, S, X, &Y, true)) return false;
            const int64_t k = kind_ == kInt4 ? 2 * W.size(1) : W.size(1);
            if (i == 0) {
                k0 = k;
                dev0 = W.device();
            } else if (k != k0 || W.device() != dev0) {
                return false;
            }
            probs[static_cast<size_t>(i)] = {W.data_ptr(), S.data_ptr(), X.data_ptr(),
                                             Y.data_ptr(), W.size(0)};
        }
        const hipStream_t stream = c10::hip::getCurrentHIPStream(dev0.index()).stream();
        const int st = grouped_(names_[static_cast<size_t>(vid)].c_str(), probs.data(),
                                static_cast<int64_t>(count), k0, stream);
        if (st == CQ_OK) return true;
        if (st == CQ_ERR_HIP)
            throw std::runtime_error(std::string(kind_ == kInt4 ? "int4gemv" : "qgemv") +
                                     " grouped launch failed (status " + std::to_string(st) +
                                     "): " + last_error_());
        return false;
    }

    bool knows(py::handle variant) const { return variant_id(variant) >= 0; }
    size_t cached() const { return cache_.size(); }
    void clear() { cache_.clear(); }

private:
    static bool all_tensors(std::initializer_list<py::handle> objs) {
        for (py::handle o : objs)
            if (!THPVariable_Check(o.ptr())) return false;
        return true;
    }

    int32_t variant_id(py::handle v) const {
        if (!PyUnicode_Check(v.ptr())) return -1;
        Py_ssize_t len = 0;
        const char* s = PyUnicode_AsUTF8AndSize(v.ptr(), &len);
        if (s == nullptr) {
            PyErr_Clear();
            return -1;
        }
        const auto it = ids_.find(std::string_view(s, static_cast<size_t>(len)));
        return it == ids_.end() ? -1 : it->second;
    }

    // INT4: W u8 (N, K/2), K % 128 == 0, scale f16 (N, K/128); INT8: W i8
    // (N, K), scale f32 (N,); both: x f16 (K,), out f16 (N,).
    bool quant_ok(const at::Tensor& w, const at::Tensor& scale, const at::Tensor& x,
                  const at::Tensor* out, bool require_gpu) const {
        const bool int4 = kind_ == kInt4;
        if (!plain(w, int4 ? at::kByte : at::kChar) || w.dim() != 2) return false;
        const int64_t n = w.size(0), k = int4 ? 2 * w.size(1) : w.size(1);
        if (n <= 0 || k <= 0 || (int4 && k % 128 != 0)) return false;
        if (!plain(scale, int4 ? at::kHalf : at::kFloat)) return false;
        if (int4 ? (scale.dim() != 2 || scale.size(0) != n || scale.size(1) != k / 128)
                 : (scale.dim() != 1 || scale.size(0) != n))
            return false;
        if (!plain(x, at::kHalf) || x.dim() != 1 || x.size(0) != k) return false;
        if (out != nullptr &&
            (!plain(*out, at::kHalf) || out->dim() != 1 || out->size(0) != n))
            return false;
        return out != nullptr ? same_device(w, {&scale, &x, out}, require_gpu)
                              : same_device(w, {&scale, &x}, require_gpu);
    }

    // W (N, K), x (K,) and out (N,), all float16 or all float32.
    bool gemv_ok(const at::Tensor& w, const at::Tensor& x, const at::Tensor* out,
                 bool require_gpu) const {
        if (!w.defined()) return false;
        const at::ScalarType dt = w.scalar_type();
        if (dt != at::kHalf && dt != at::kFloat) return false;
        if (!plain(w, dt) || w.dim() != 2 || w.size(0) <= 0 || w.size(1) <= 0) return false;
        if (!plain(x, dt) || x.dim() != 1 || x.size(0) != w.size(1)) return false;
        if (out != nullptr && (!plain(*out, dt) || out->dim() != 1 || out->size(0) != w.size(0)))
            return false;
        return out != nullptr ? same_device(w, {&x, out}, require_gpu)
                              : same_device(w, {&x}, require_gpu);
    }

    int op_code(const at::Tensor& w) const {
        if (kind_ == kInt4) return CQ_OP_INT4GEMV;
        if (kind_ == kQ8) return CQ_OP_QGEMV;
        return w.scalar_type() == at::kFloat ? CQ_OP_GEMV_F32 : CQ_OP_GEMV_F16;
    }

    bool run(int32_t vid, const at::Tensor& w, const void* scale, const at::Tensor& x,
             const at::Tensor& out) {
        const int op = op_code(w);
        const int64_t n = w.size(0);
        const int64_t k = kind_ == kInt4 ? 2 * w.size(1) : w.size(1);
        const Key key{w.data_ptr(), scale, x.data_ptr(), out.data_ptr(), n, k, vid, op};
        auto it = cache_.find(key);
        if (it == cache_.end()) {
            cq_prepared_t rec;
            if (prepare_(op, names_[static_cast<size_t>(vid)].c_str(), key.w, key.s,
                         key.x, const_cast<void*>(key.y), n, k, &rec) != CQ_OK)
                return false;
            if (cache_.size() >= capacity_) cache_.clear();
            it = cache_.emplace(key, rec).first;
        }
        const hipStream_t stream =
            c10::hip::getCurrentHIPStream(w.device().index()).stream();
        const int st = launch_(&it->second, stream);
        if (st != CQ_OK) {
            const char* op_name = kind_ == kInt4 ? "int4gemv" : kind_ == kQ8 ? "qgemv" : "gemv";
            throw std::runtime_error(std::string(op_name) + " launch failed (status " +
                                     std::to_string(st) + "): " + last_error_());
        }
        return true;
    }

    int kind_;
    PrepareFn prepare_;
    LaunchFn launch_;
    ErrorFn last_error_;
    GroupedFn grouped_;
    size_t capacity_;
    std::vector<std::string> names_;
    std::unordered_map<std::string_view, int32_t> ids_;
    std::unordered_map<Key, cq_prepared_t, KeyHash> cache_;
};

}  // namespace

PYBIND11_MODULE(_cqfast, m) {
    m.doc() = "Checked-once launch path of the eager GEMV API (see ext.py)";
    m.attr("src_hash") = CQ_SRC_HASH;
    m.attr("abi_stamp") = CQ_FAST_ABI;   // torch version, C++ ABI, g++ flags
    py::class_<Launcher>(m, "Launcher")
        .def(py::init<int, const std::vector<std::string>&, uintptr_t, uintptr_t,
                      uintptr_t, int64_t, uintptr_t>(),
             py::arg("kind"), py::arg("names"), py::arg("prepare"), py::arg("launch"),
             py::arg("last_error"), py::arg("capacity"), py::arg("grouped") = 0)
        .def("accepts", &Launcher::accepts)
        .def("gemv_accepts", &Launcher::gemv_accepts)
        .def("into", &Launcher::into)
        .def("forward", &Launcher::forward)
        .def("gemv_into", &Launcher::gemv_into)
        .def("gemv_forward", &Launcher::gemv_forward)
        .def("grouped", &Launcher::grouped)
        .def("knows", &Launcher::knows)
        .def("cached", &Launcher::cached)
        .def("clear", &Launcher::clear);
}
