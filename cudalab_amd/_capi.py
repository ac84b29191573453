"""ctypes binding of `libcdnaqgemv.so` (declarations in include/cdnaqgemv.h).

Loading happens once, on first use.  There is no fallback: if the library
is missing or does not export the declared symbols, every entry point
raises, so no GEMV can silently run anywhere but in the HIP kernels.

The library must be loaded after `import torch` so that its HIP runtime
dependency (soname libamdhip64.so.7) binds to the runtime torch already
loaded: streams and device pointers handed over from torch are then valid
in the library.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from .build import FAST_NAME, LIB_PATH, fast_abi_stamp, fast_module_path, source_hash

CQ_OK = 0
CQ_ERR_UNKNOWN_VARIANT = 1
CQ_ERR_INVALID_ARG = 2
CQ_ERR_HIP = 3
CQ_ERR_BUFFER_TOO_SMALL = 4

CQ_OP_INT4GEMV = 0
CQ_OP_QGEMV = 1
CQ_OP_GEMV_F16 = 2
CQ_OP_GEMV_F32 = 3

CQ_DTYPE_F16 = 0
CQ_DTYPE_F32 = 1

# quantizer scale forms: amax / qmax (torch on the CPU) or amax * fl(1/qmax)
# (torch on a GPU)
CQ_SCALE_DIV = 0
CQ_SCALE_RCP = 1

# rows longer than this run the K-tiled kernels (cq_internal.h kMaxWaveK)
MAX_UNTILED_K = 16384

CQ_LIST_NORMAL = 0
CQ_LIST_ALL = 1
CQ_LIST_QUARANTINED = 2
CQ_LIST_ALIASES = 3

# operator ids by name; "gemv" lists its (dtype-independent) registry
# through the fp16 id
OPS = {"int4gemv": CQ_OP_INT4GEMV, "qgemv": CQ_OP_QGEMV,
       "gemv": CQ_OP_GEMV_F16, "gemv_f16": CQ_OP_GEMV_F16,
       "gemv_f32": CQ_OP_GEMV_F32}


class CqTiming(ctypes.Structure):
    _fields_ = [
        ("warmup", ctypes.c_int64),
        ("n_windows", ctypes.c_int64),
        ("launches_per_window", ctypes.c_int64),
        ("median_us", ctypes.c_double),
        ("min_us", ctypes.c_double),
        ("max_us", ctypes.c_double),
        ("mean_us", ctypes.c_double),
    ]


class CqProblem(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("x", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("n", ctypes.c_int64),
    ]


class CqPrepared(ctypes.Structure):
    """cq_prepared_t: a launch resolved by cq_prepare (opaque)."""
    _fields_ = [("opaque", ctypes.c_uint64 * 12)]


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_cstr = ctypes.c_char_p

# name -> (restype, argtypes); must match include/cdnaqgemv.h
SIGNATURES = {
    "cq_int4gemv": (ctypes.c_int, [_cstr, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "cq_qgemv": (ctypes.c_int, [_cstr, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "cq_gemv": (ctypes.c_int, [_cstr, ctypes.c_int, _vp, _vp, _vp, _i64, _i64,
                               _vp]),
    "cq_int4gemv_grouped": (ctypes.c_int, [_cstr, ctypes.POINTER(CqProblem),
                                           _i64, _i64, _vp]),
    "cq_qgemv_grouped": (ctypes.c_int, [_cstr, ctypes.POINTER(CqProblem),
                                        _i64, _i64, _vp]),
    "cq_int4_quantize": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64,
                                        ctypes.c_int, _vp]),
    "cq_q8_quantize": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64,
                                      ctypes.c_int, _vp]),
    "cq_quantize_vectorized": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _i64,
                                              _i64]),
    "cq_native_timing": (ctypes.c_int, [
        ctypes.c_int, _cstr, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64,
        _i64, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(CqTiming)]),
    "cq_pool_timing": (ctypes.c_int, [
        ctypes.c_int, _cstr, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
        ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i64, _i64, _i64, _vp,
        _i64, ctypes.c_double, ctypes.c_double, _i64,
        ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_double),
        ctypes.POINTER(ctypes.c_double)]),
    "cq_read_ceiling": (ctypes.c_int, [ctypes.POINTER(_vp), _i64, _i64, _vp,
                                       _vp, _i64, ctypes.c_double,
                                       ctypes.c_double, _i64,
                                       ctypes.POINTER(ctypes.c_double)]),
    "cq_launch_floor": (ctypes.c_int, [_i64, ctypes.c_int, _vp, _vp, _i64,
                                       ctypes.c_double, ctypes.c_double, _i64,
                                       ctypes.POINTER(ctypes.c_double)]),
    "cq_int4_timeline": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp),
                                        ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                        ctypes.POINTER(_vp), _i64, _i64, _i64, _vp,
                                        _i64, ctypes.c_double, ctypes.c_double,
                                        _i64, _vp, _i64, ctypes.POINTER(_i64),
                                        ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_double)]),
    "cq_variants": (ctypes.c_int, [ctypes.c_int, ctypes.c_int,
                                   ctypes.c_char_p, ctypes.c_size_t]),
    "cq_vec_contract_ok": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _i64]),
    "cq_describe_launch": (ctypes.c_int, [ctypes.c_int, _cstr, _i64, _i64,
                                          _vp, _vp, ctypes.c_char_p,
                                          ctypes.c_size_t]),
    "cq_prepare": (ctypes.c_int, [ctypes.c_int, _cstr, _vp, _vp, _vp, _vp,
                                  _i64, _i64, ctypes.POINTER(CqPrepared)]),
    "cq_launch_prepared": (ctypes.c_int, [_vp, _vp]),
    "cq_last_error": (ctypes.c_char_p, []),
    "cq_version": (ctypes.c_char_p, []),
}

_lib = None
_lock = threading.Lock()


class LibraryMissing(RuntimeError):
    pass


class StaleLibrary(RuntimeError):
    """The built library's source stamp differs from the tree's sources."""


def lib_path() -> Path:
    return LIB_PATH


def load():
    """Load the library once and declare every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (bind libamdhip64 to torch's runtime first)
        if not LIB_PATH.exists():
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -m cudalab_amd.build` "
                "(or __graft_entry__.build()). The HIP library is the only "
                "implementation of this path: there is no CPU fallback.")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if not exported
            fn.restype = res
            fn.argtypes = args
        built = library_stamp(lib)
        tree = source_hash()
        if built != tree:
            raise StaleLibrary(
                f"{LIB_PATH} was built from other sources than the tree holds "
                f"(library src={built}, tree src={tree}); rebuild it with "
                "`python -m cudalab_amd.build` (or __graft_entry__.build()).")
        _lib = lib
        return lib


_fast = None


def fast_module():
    """The eager fast-path module (`_cqfast`, built beside the library from
    csrc/cq_pyfast.cpp), loaded once; refused, like the library, when
    missing, built from other sources than the tree holds, or built against
    another torch (version, C++ ABI flag or g++ flags: `fast_abi_stamp`)."""
    global _fast
    if _fast is not None:
        return _fast
    load()
    with _lock:
        if _fast is not None:
            return _fast
        import importlib.util
        path = fast_module_path()
        if not path.exists():
            raise LibraryMissing(
                f"{path} is not built; run `python -m cudalab_amd.build` "
                "(or __graft_entry__.build()).")
        spec = importlib.util.spec_from_file_location(FAST_NAME, path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if mod.src_hash != source_hash():
            raise StaleLibrary(
                f"{path} was built from other sources than the tree holds "
                f"(module src={mod.src_hash}, tree src={source_hash()}); rebuild "
                "it with `python -m cudalab_amd.build`.")
        abi = getattr(mod, "abi_stamp", "unstamped")
        if abi != fast_abi_stamp():
            raise StaleLibrary(
                f"{path} was built against another torch or with other flags "
                f"(module {abi}, this process {fast_abi_stamp()}); rebuild it "
                "with `python -m cudalab_amd.build`.")
        _fast = mod
        return mod


def entry_address(name: str) -> int:
    """Address of a library entry point (for the fast-path module, which
    calls the same loaded library)."""
    return ctypes.cast(getattr(load(), name), ctypes.c_void_p).value


def library_stamp(lib) -> str:
    """The source stamp compiled into a loaded library ("src=..." at the
    end of cq_version())."""
    v = lib.cq_version().decode("ascii", "replace")
    return v.rsplit("src=", 1)[1] if "src=" in v else "unstamped"


def last_error() -> str:
    return load().cq_last_error().decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    if status != CQ_OK:
        raise RuntimeError(f"{what} failed (status {status}): {last_error()}")


def _string_call(fn, *args) -> str:
    need = fn(*args, None, 0)
    if need < 0:
        raise RuntimeError(f"{fn.__name__} failed (status {need}): "
                           f"{last_error()}")
    buf = ctypes.create_string_buffer(need)
    got = fn(*args, buf, need)
    if got != need:
        raise RuntimeError(f"{fn.__name__}: size changed ({need} -> {got})")
    return buf.value.decode("utf-8")


def variant_list(op: str, which: int = CQ_LIST_NORMAL) -> list[str]:
    s = _string_call(load().cq_variants, OPS[op], which)
    return [v for v in s.split("\n") if v]


def aliases(op: str) -> dict[str, str]:
    out = {}
    for line in variant_list(op, CQ_LIST_ALIASES):
        a, t = line.split("=", 1)
        out[a] = t
    return out


def describe_launch(op: str, variant: str, n: int, k: int, w_ptr: int,
                    x_ptr: int) -> dict:
    s = _string_call(load().cq_describe_launch, OPS[op],
                     variant.encode(), n, k, w_ptr, x_ptr)
    return parse_launch_line(s)


def parse_launch_line(s: str) -> dict:
    """Parse cq_describe_launch's "key=value ... why=<free text>" line."""
    head, why = s.split(" why=", 1)
    out = dict(tok.split("=", 1) for tok in head.split(" "))
    out["why"] = why
    return out


def vec_contract_ok(op: str, w_ptr: int, x_ptr: int, k: int) -> bool:
    return bool(load().cq_vec_contract_ok(OPS[op], w_ptr, x_ptr, k))


def version() -> str:
    return load().cq_version().decode()
