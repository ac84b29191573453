"""Python extension objects for the two operators, over the C ABI.

Drop-in for the reference's per-operator pybind modules
(kernels/int4gemv/bindings.cpp:287-316, kernels/qgemv/bindings.cpp:280-308):
the same functions (`forward`, `forward_into`, `native_timing`, `variants`,
`all_variants`, `quarantined_variants`), the same argument meaning, the same
validation order, and the same message substrings, which callers match
(cudalab/int4gemv_negative.py:108-318, cudalab/qgemv_negative.py:103-300).
Every check runs on host metadata before anything is launched and raises
RuntimeError (the type TORCH_CHECK surfaced as).

What differs by design: the checks that raise live here, in Python, where
the CPU test suite can reach them; the C layer receives plain pointers and
sizes and picks the kernel (vectorized or scalar fallback) from alignment.
Launches go on the current torch stream of the weights' device.

`forward`, `forward_into` and `forward_grouped` first offer the call to the
fast path (csrc/cq_pyfast.cpp): one C++ call that applies the same
acceptance rule to the tensors' metadata, looks the launch up in a cache of
launches prepared once by cq_prepare (keyed by variant, operand addresses
and sizes, so a cached launch is exactly what preparing again would give)
and enqueues it; a grouped call goes to the library's grouped entry point
directly.  It launches nothing for a call it does not accept, and the
checked path below then runs and raises in the reference's order.  On
MI355X this took an INT4 forward_into from 7.0-8.2 us of host time to
3.0-3.2 us, within 0.1-0.7 us of hipLaunchKernel itself (2.2-3.1 us
depending on the host).
"""
from __future__ import annotations

import ctypes
import warnings
from typing import Optional

import torch

from . import _capi


def _on_device(dev: torch.device, call):
    """call(stream) with `stream` the raw handle of `dev`'s current HIP
    stream and `dev` the current device (a launch must be issued with its
    stream's device current).  The usual case -- `dev` already current --
    takes the raw handle directly, about 3 us per call cheaper than entering
    torch.cuda.device and building a Stream object."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if torch.cuda.current_device() == idx:
        return call(torch._C._cuda_getCurrentRawStream(idx))
    with torch.cuda.device(idx):
        return call(torch._C._cuda_getCurrentRawStream(idx))

NATIVE_TIMING_NOTE = (
    "native kernel-loop caliber: back-to-back launches from C++ between two "
    "HIP events on the current stream, window time / launches; no Python "
    "boundary inside the window (distinct from the API-path caliber and from "
    "the profiler's per-dispatch kernel duration)")


# prepared launches kept per operator (the cache is cleared when full)
FAST_CACHE_ENTRIES = 4096
_FAST_KIND = {"int4gemv": 0, "qgemv": 1, "gemv": 2}


_GROUPED_ENTRY = {"int4gemv": "cq_int4gemv_grouped", "qgemv": "cq_qgemv_grouped"}


class _DeclineAll:
    """Stand-in for the fast-path launcher when its module is missing, stale
    or fails to import: it accepts no call, so every call takes the checked
    path (which launches the same HIP kernels through the library)."""

    def accepts(self, *args) -> bool:
        return False

    gemv_accepts = knows = into = gemv_into = grouped = accepts

    def forward(self, *args):
        return None

    gemv_forward = forward

    def cached(self) -> int:
        return 0

    def clear(self) -> None:
        pass


_fast_warned = False


def _fast_launcher(op: str, names: list[str]):
    """The fast-path launcher of `op`, or a launcher that declines every
    call (with one warning per process) when the fast-path module cannot
    be used; the checked path is complete without it."""
    global _fast_warned
    grouped = _GROUPED_ENTRY.get(op)
    try:
        mod = _capi.fast_module()
    except (_capi.LibraryMissing, _capi.StaleLibrary, ImportError, OSError) as e:
        if not _fast_warned:
            _fast_warned = True
            warnings.warn(f"eager fast path unavailable, every call takes the "
                          f"checked path: {e}", RuntimeWarning, stacklevel=3)
        return _DeclineAll()
    return mod.Launcher(
        _FAST_KIND[op], names, _capi.entry_address("cq_prepare"),
        _capi.entry_address("cq_launch_prepared"),
        _capi.entry_address("cq_last_error"), FAST_CACHE_ENTRIES,
        _capi.entry_address(grouped) if grouped else 0)


def _fail(msg: str) -> None:
    raise RuntimeError(msg)


def _same_device(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.device == b.device


class _OpExt:
    """Common machinery; subclasses define the operator and its checks."""

    op: str = ""

    def __init__(self) -> None:
        self._lib = _capi.load()
        self._normal = _capi.variant_list(self.op, _capi.CQ_LIST_NORMAL)
        self._all = _capi.variant_list(self.op, _capi.CQ_LIST_ALL)
        self._quar = _capi.variant_list(self.op, _capi.CQ_LIST_QUARANTINED)
        self._aliases = _capi.aliases(self.op)
        self._fn = (self._lib.cq_int4gemv if self.op == "int4gemv"
                    else self._lib.cq_qgemv)
        self._grouped_fn = (self._lib.cq_int4gemv_grouped
                            if self.op == "int4gemv"
                            else self._lib.cq_qgemv_grouped)
        self._fast = _fast_launcher(self.op, self._all + sorted(self._aliases))

    # ---- registry (bindings.cpp variant lists) ----
    def variants(self) -> list[str]:
        """Dispatchable variants, sorted; quarantined ones excluded."""
        return list(self._normal)

    def all_variants(self) -> list[str]:
        """Every registered variant, quarantined ones included, sorted."""
        return list(self._all)

    def quarantined_variants(self) -> list[str]:
        return list(self._quar)

    def aliases(self) -> dict[str, str]:
        """Reference variant names accepted as aliases -> target variant."""
        return dict(self._aliases)

    def resolve(self, name: str) -> str:
        return self._aliases.get(name, name)

    def _unknown_variant_msg(self, name: str) -> str:
        s = (f"未知 {self.op} 变体 '{name}'。正常可用: "
             + " ".join(self._normal) + " ")
        if self._quar:
            s += ("；被隔离（NOT_FOR_NORMAL_DISPATCH）: " + " ".join(self._quar)
                  + " （显式命名仍可调用，属受控历史审计入口）")
        s += f"(unknown {self.op} variant)"
        return s

    def _lookup(self, name: str) -> str:
        if not isinstance(name, str):
            _fail(self._unknown_variant_msg(str(name)))
        if name in self._all or name in self._aliases:
            return name
        _fail(self._unknown_variant_msg(name))

    # ---- subclass hooks ----
    def _validate_w(self, W: torch.Tensor) -> None:
        raise NotImplementedError

    def _validate_scale(self, W: torch.Tensor, scale: torch.Tensor) -> None:
        raise NotImplementedError

    def _validate_x(self, W: torch.Tensor, x: torch.Tensor) -> None:
        raise NotImplementedError

    def _k(self, W: torch.Tensor) -> int:
        raise NotImplementedError

    def _w_name(self) -> str:
        raise NotImplementedError

    def _validate_out(self, W: torch.Tensor, out: torch.Tensor) -> None:
        if out.dim() != 1:
            _fail(f"out 必须是 1 维 (N,)，实际 {out.dim()} 维 (out must be 1-D)")
        if out.size(0) != W.size(0):
            _fail(f"out 长度必须等于 N: out={out.size(0)} N={W.size(0)} "
                  "(out length must equal N)")
        if out.dtype != torch.float16:
            _fail(f"out 必须是 float16，实际 {out.dtype} (out must be float16)")
        if not out.is_contiguous():
            _fail("out 必须是连续内存 (out must be contiguous)")
        if not out.is_cuda:
            _fail("out 必须是 CUDA 张量 (out must be a GPU tensor)")
        if not _same_device(out, W):
            _fail(f"out 必须与 {self._w_name()} 在同一 CUDA 设备上 "
                  "(out must be on the weights' device)")

    def _validate_inputs(self, W, scale, x) -> None:
        self._validate_w(W)
        self._validate_scale(W, scale)
        self._validate_x(W, x)

    # ---- launch ----
    def _launch(self, variant: str, W, scale, x, out) -> None:
        st = _on_device(W.device, lambda stream: self._fn(
            variant.encode(), W.data_ptr(), scale.data_ptr(), x.data_ptr(),
            out.data_ptr(), W.size(0), self._k(W), stream))
        if st != _capi.CQ_OK:
            _fail(f"{self.op} launch failed (status {st}): "
                  f"{_capi.last_error()}")

    def forward(self, variant: str, W: torch.Tensor, scale: torch.Tensor,
                x: torch.Tensor) -> torch.Tensor:
        """y = W_dequant @ x into a newly allocated fp16 (N,) tensor."""
        y = self._fast.forward(variant, W, scale, x)
        if y is not None:
            return y
        self._lookup(variant)
        self._validate_inputs(W, scale, x)
        out = torch.empty(W.size(0), dtype=torch.float16, device=W.device)
        self._launch(variant, W, scale, x, out)
        return out

    def forward_into(self, variant: str, W: torch.Tensor,
                     scale: torch.Tensor, x: torch.Tensor,
                     out: torch.Tensor) -> None:
        """Same as forward, writing into a preallocated `out` (N,) fp16."""
        if self._fast.into(variant, W, scale, x, out):
            return
        self._lookup(variant)
        self._validate_inputs(W, scale, x)
        self._validate_out(W, out)
        self._launch(variant, W, scale, x, out)

    def forward_grouped(self, variant: str, problems) -> None:
        """Several independent GEMVs sharing K, in as few launches as the
        variant allows (one per 8 problems for the CDNA4 LDS variants).
        `problems` is a sequence of (W, scale, x, out) tuples, each checked
        exactly as forward_into checks its arguments; every `out` is then
        bit-identical to forward_into(variant, W, scale, x, out).  No
        counterpart in the reference (its modules launch one problem at a
        time)."""
        if self._fast.grouped(variant, problems):
            return
        self._lookup(variant)
        problems = list(problems)
        if not problems:
            _fail("problems 不能为空 (problems must be a non-empty list)")
        K = None
        dev = None
        for (W, scale, x, out) in problems:
            self._validate_inputs(W, scale, x)
            self._validate_out(W, out)
            if K is None:
                K, dev = self._k(W), W.device
            elif self._k(W) != K:
                _fail(f"分组调用的所有问题必须有相同的 K: {K} vs {self._k(W)} "
                      "(all problems of a grouped call must share K)")
            elif W.device != dev:
                _fail("分组调用的所有问题必须在同一 CUDA 设备上 "
                      "(all problems of a grouped call must be on one device)")
        arr = (_capi.CqProblem * len(problems))()
        for i, (W, scale, x, out) in enumerate(problems):
            arr[i].w = W.data_ptr()
            arr[i].scale = scale.data_ptr()
            arr[i].x = x.data_ptr()
            arr[i].y = out.data_ptr()
            arr[i].n = W.size(0)
        st = _on_device(dev, lambda stream: self._grouped_fn(
            variant.encode(), arr, len(problems), K, stream))
        if st != _capi.CQ_OK:
            _fail(f"{self.op} grouped launch failed (status {st}): "
                  f"{_capi.last_error()}")

    def native_timing(self, variant: str, W: torch.Tensor,
                      scale: torch.Tensor, x: torch.Tensor,
                      out: torch.Tensor, warmup: int = 200,
                      n_windows: int = 10,
                      launches_per_window: int = 64) -> dict:
        """Native kernel-loop timing (bindings.cpp:180-253 semantics)."""
        self._lookup(variant)
        if warmup < 0:
            _fail(f"warmup 必须 >= 0，实际 {warmup}")
        if n_windows < 1:
            _fail(f"n_windows 必须 >= 1，实际 {n_windows}")
        if launches_per_window < 1:
            _fail(f"launches_per_window 必须 >= 1，实际 {launches_per_window}")
        self._validate_inputs(W, scale, x)
        self._validate_out(W, out)
        win = (ctypes.c_double * n_windows)()
        res = _capi.CqTiming()
        st = _on_device(W.device, lambda stream: self._lib.cq_native_timing(
                _capi.OPS[self.op], variant.encode(), W.data_ptr(),
                scale.data_ptr(), x.data_ptr(), out.data_ptr(), W.size(0),
                self._k(W), stream, warmup, n_windows, launches_per_window,
                win, ctypes.byref(res)))
        if st != _capi.CQ_OK:
            _fail(f"native_timing failed (status {st}): {_capi.last_error()}")
        return {
            "variant": variant,
            "warmup": int(warmup),
            "n_windows": int(n_windows),
            "launches_per_window": int(launches_per_window),
            "window_median_us": [float(v) for v in win],
            "median_us": res.median_us,
            "min_us": res.min_us,
            "max_us": res.max_us,
            "mean_us": res.mean_us,
            "note": NATIVE_TIMING_NOTE,
        }

    def describe(self, variant: str, W: torch.Tensor,
                 x: torch.Tensor) -> dict:
        """Kernel and launch shape the library would use (no launch)."""
        self._lookup(variant)
        s = _capi._string_call(self._lib.cq_describe_launch,
                               _capi.OPS[self.op], variant.encode(),
                               W.size(0), self._k(W), W.data_ptr(),
                               x.data_ptr())
        return _capi.parse_launch_line(s)

    def contract_ok(self, W: torch.Tensor, x: torch.Tensor) -> bool:
        """Host predicate of the vector contract for these tensors."""
        return _capi.vec_contract_ok(self.op, W.data_ptr(), x.data_ptr(),
                                     self._k(W))


class Int4gemvExt(_OpExt):
    """W4A16 INT4 GEMV: W_packed u8 (N,K/2), scale f16 (N,K/128), x f16 (K,).

    Checks in the order of kernels/int4gemv/bindings.cpp:60-121."""

    op = "int4gemv"

    def _w_name(self) -> str:
        return "W_packed"

    def _k(self, W: torch.Tensor) -> int:
        return 2 * W.size(1)

    def _validate_w(self, Wp: torch.Tensor) -> None:
        if Wp.dim() != 2:
            _fail(f"W_packed 必须是 2 维 (N, K/2)，实际 {Wp.dim()} 维 "
                  "(W_packed must be 2-D)")
        if Wp.size(0) <= 0:
            _fail(f"N 必须 > 0，实际 {Wp.size(0)} (N must be > 0)")
        if Wp.size(1) <= 0:
            _fail(f"K/2 必须 > 0，实际 {Wp.size(1)} (K/2 must be > 0)")
        if Wp.dtype != torch.uint8:
            _fail(f"W_packed 必须是 uint8，实际 {Wp.dtype} "
                  "(W_packed must be uint8)")
        K = 2 * Wp.size(1)
        if K % 128 != 0:
            _fail(f"K 必须可被 128 整除（group_size=128 合同）, 实际 K={K} "
                  "(K must be divisible by 128)")
        if not Wp.is_contiguous():
            _fail("W_packed 必须是连续内存 (W_packed must be contiguous)")
        if not Wp.is_cuda:
            _fail("W_packed 必须是 CUDA 张量 (W_packed must be a GPU tensor)")

    def _validate_scale(self, Wp: torch.Tensor, scale: torch.Tensor) -> None:
        N, K = Wp.size(0), 2 * Wp.size(1)
        if scale.dim() != 2:
            _fail(f"scale 必须是 2 维 (N, K/128)，实际 {scale.dim()} 维 "
                  "(scale must be 2-D)")
        if scale.size(0) != N:
            _fail(f"scale 行数必须等于 N: scale={scale.size(0)} N={N} "
                  "(scale rows must equal N)")
        if scale.size(1) != K // 128:
            _fail(f"scale 组数必须等于 K/128（invalid group count）: "
                  f"scale={scale.size(1)} K/128={K // 128}")
        if scale.dtype != torch.float16:
            _fail(f"scale 必须是 float16, 实际 {scale.dtype} "
                  "(scale must be float16)")
        if not scale.is_contiguous():
            _fail("scale 必须是连续内存 (scale must be contiguous)")
        if not scale.is_cuda:
            _fail("scale 必须是 CUDA 张量 (scale must be a GPU tensor)")
        if not _same_device(scale, Wp):
            _fail("scale 必须与 W_packed 在同一 CUDA 设备上 "
                  "(scale must be on W_packed's device)")

    def _validate_x(self, Wp: torch.Tensor, x: torch.Tensor) -> None:
        K = 2 * Wp.size(1)
        if x.dim() != 1:
            _fail(f"x 必须是 1 维 (K,)，实际 {x.dim()} 维 (x must be 1-D)")
        if x.size(0) != K:
            _fail(f"x 长度必须等于 K: x={x.size(0)} K={K} "
                  "(x length must equal K)")
        if x.dtype != torch.float16:
            _fail(f"x 必须是 float16, 实际 {x.dtype} (x must be float16)")
        if not x.is_contiguous():
            _fail("x 必须是连续内存 (x must be contiguous)")
        if not x.is_cuda:
            _fail("x 必须是 CUDA 张量 (x must be a GPU tensor)")
        if not _same_device(x, Wp):
            _fail("x 必须与 W_packed 在同一 CUDA 设备上 "
                  "(x must be on W_packed's device)")


class QgemvExt(_OpExt):
    """W8A16 INT8 GEMV: W_q i8 (N,K), scale f32 (N,), x f16 (K,).

    Checks in the order of kernels/qgemv/bindings.cpp:65-121."""

    op = "qgemv"

    def _w_name(self) -> str:
        return "W_q"

    def _k(self, W: torch.Tensor) -> int:
        return W.size(1)

    def _validate_w(self, Wq: torch.Tensor) -> None:
        if Wq.dim() != 2:
            _fail(f"W_q 必须是 2 维 (N, K)，实际 {Wq.dim()} 维 (W_q must be 2-D)")
        if Wq.size(0) <= 0:
            _fail(f"N 必须 > 0，实际 {Wq.size(0)} (N must be > 0)")
        if Wq.size(1) <= 0:
            _fail(f"K 必须 > 0，实际 {Wq.size(1)} (K must be > 0)")
        if Wq.dtype != torch.int8:
            _fail(f"W_q 必须是 int8，实际 {Wq.dtype} (W_q must be int8)")
        if not Wq.is_contiguous():
            _fail("W_q 必须是连续内存 (W_q must be contiguous)")
        if not Wq.is_cuda:
            _fail("W_q 必须是 CUDA 张量 (W_q must be a GPU tensor)")

    def _validate_scale(self, Wq: torch.Tensor, scale: torch.Tensor) -> None:
        if scale.dim() != 1:
            _fail(f"scale 必须是 1 维 (N,)，实际 {scale.dim()} 维 "
                  "(scale must be 1-D)")
        if scale.size(0) != Wq.size(0):
            _fail(f"scale 长度必须等于 N: scale={scale.size(0)} N={Wq.size(0)} "
                  "(scale length must equal N)")
        if scale.dtype != torch.float32:
            _fail(f"scale 必须是 float32，实际 {scale.dtype} "
                  "(scale must be float32)")
        if not scale.is_contiguous():
            _fail("scale 必须是连续内存 (scale must be contiguous)")
        if not scale.is_cuda:
            _fail("scale 必须是 CUDA 张量 (scale must be a GPU tensor)")
        if not _same_device(scale, Wq):
            _fail("scale 必须与 W_q 在同一 CUDA 设备上 "
                  "(scale must be on W_q's device)")

    def _validate_x(self, Wq: torch.Tensor, x: torch.Tensor) -> None:
        if x.dim() != 1:
            _fail(f"x 必须是 1 维 (K,)，实际 {x.dim()} 维 (x must be 1-D)")
        if x.size(0) != Wq.size(1):
            _fail(f"x 长度必须等于 K: x={x.size(0)} K={Wq.size(1)} "
                  "(x length must equal K)")
        if x.dtype != torch.float16:
            _fail(f"x 必须是 float16, 实际 {x.dtype} (x must be float16)")
        if not x.is_contiguous():
            _fail("x 必须是连续内存 (x must be contiguous)")
        if not x.is_cuda:
            _fail("x 必须是 CUDA 张量 (x must be a GPU tensor)")
        if not _same_device(x, Wq):
            _fail("x 必须与 W_q 在同一 CUDA 设备上 "
                  "(x must be on W_q's device)")


class GemvExt(_OpExt):
    """FP16/FP32 GEMV: W (N,K), x (K,), out (N,), all float16 or all
    float32; FP32 accumulation (kernels/gemv/gemv_common.h:1-79).

    Same methods as the reference's gemv module
    (kernels/gemv/bindings.cpp:310-336) with two-tensor signatures:
    forward(variant, W, x), forward_into(variant, W, x, out),
    native_timing(variant, W, x, out, ...).  Checks in the order of
    kernels/gemv/bindings.cpp:87-125."""

    op = "gemv"

    def __init__(self) -> None:
        super().__init__()
        self._fn = self._lib.cq_gemv
        self._grouped_fn = None

    def _w_name(self) -> str:
        return "W"

    def _k(self, W: torch.Tensor) -> int:
        return W.size(1)

    @staticmethod
    def _op_id(W: torch.Tensor) -> int:
        return (_capi.CQ_OP_GEMV_F32 if W.dtype == torch.float32
                else _capi.CQ_OP_GEMV_F16)

    def _validate_w(self, W: torch.Tensor) -> None:
        if W.dim() != 2:
            _fail(f"W 必须是 2 维 (N, K)，实际 {W.dim()} 维 (W must be 2-D)")
        if W.size(0) <= 0:
            _fail(f"N 必须 > 0，实际 {W.size(0)} (N must be > 0)")
        if W.size(1) <= 0:
            _fail(f"K 必须 > 0，实际 {W.size(1)} (K must be > 0)")
        if W.dtype not in (torch.float16, torch.float32):
            _fail(f"仅支持 float16 / float32，实际 {W.dtype} "
                  "(only float16 / float32)")
        if not W.is_contiguous():
            _fail("W 必须是连续内存 (W must be contiguous)")
        if not W.is_cuda:
            _fail("W 必须是 CUDA 张量 (W must be a GPU tensor)")

    def _validate_x(self, W: torch.Tensor, x: torch.Tensor) -> None:
        if x.dim() != 1:
            _fail(f"x 必须是 1 维 (K,)，实际 {x.dim()} 维 (x must be 1-D)")
        if x.size(0) != W.size(1):
            _fail(f"x 长度必须等于 K: x={x.size(0)} K={W.size(1)} "
                  "(x length must equal K)")
        if x.dtype != W.dtype:
            _fail(f"x 的 dtype 必须与 W 一致: x={x.dtype} W={W.dtype} "
                  "(x dtype must match W)")
        if not x.is_contiguous():
            _fail("x 必须是连续内存 (x must be contiguous)")
        if not x.is_cuda:
            _fail("x 必须是 CUDA 张量 (x must be a GPU tensor)")
        if not _same_device(x, W):
            _fail("x 必须与 W 在同一 CUDA 设备上 (x must be on W's device)")

    def _validate_out(self, W: torch.Tensor, out: torch.Tensor) -> None:
        if out.dim() != 1:
            _fail(f"out 必须是 1 维 (N,)，实际 {out.dim()} 维 (out must be 1-D)")
        if out.size(0) != W.size(0):
            _fail(f"out 长度必须等于 N: out={out.size(0)} N={W.size(0)} "
                  "(out length must equal N)")
        if out.dtype != W.dtype:
            _fail(f"out 的 dtype 必须与 W 一致: out={out.dtype} W={W.dtype} "
                  "(out dtype must match W)")
        if not out.is_contiguous():
            _fail("out 必须是连续内存 (out must be contiguous)")
        if not out.is_cuda:
            _fail("out 必须是 CUDA 张量 (out must be a GPU tensor)")
        if not _same_device(out, W):
            _fail("out 必须与 W 在同一 CUDA 设备上 (out must be on W's device)")

    def _launch2(self, variant: str, W, x, out) -> None:
        dev = W.device
        dt = (_capi.CQ_DTYPE_F32 if W.dtype == torch.float32
              else _capi.CQ_DTYPE_F16)
        st = _on_device(dev, lambda stream: self._fn(
            variant.encode(), dt, W.data_ptr(), x.data_ptr(), out.data_ptr(),
            W.size(0), W.size(1), stream))
        if st != _capi.CQ_OK:
            _fail(f"gemv launch failed (status {st}): {_capi.last_error()}")

    def forward(self, variant: str, W: torch.Tensor,  # type: ignore[override]
                x: torch.Tensor) -> torch.Tensor:
        """y = W @ x (FP32 accumulation) into a new (N,) tensor of W's dtype."""
        y = self._fast.gemv_forward(variant, W, x)
        if y is not None:
            return y
        self._lookup(variant)
        self._validate_w(W)
        self._validate_x(W, x)
        out = torch.empty(W.size(0), dtype=W.dtype, device=W.device)
        self._launch2(variant, W, x, out)
        return out

    def forward_into(self, variant: str, W: torch.Tensor,  # type: ignore[override]
                     x: torch.Tensor, out: torch.Tensor) -> None:
        if self._fast.gemv_into(variant, W, x, out):
            return
        self._lookup(variant)
        self._validate_w(W)
        self._validate_x(W, x)
        self._validate_out(W, out)
        self._launch2(variant, W, x, out)

    def forward_grouped(self, variant, problems):  # type: ignore[override]
        _fail("gemv 不提供分组调用 (grouped calls exist for int4gemv and qgemv)")

    def native_timing(self, variant: str, W: torch.Tensor,  # type: ignore[override]
                      x: torch.Tensor, out: torch.Tensor, warmup: int = 200,
                      n_windows: int = 10,
                      launches_per_window: int = 64) -> dict:
        """Native kernel-loop timing (kernels/gemv/bindings.cpp:194-276
        semantics)."""
        self._lookup(variant)
        if warmup < 0:
            _fail(f"warmup 必须 >= 0，实际 {warmup}")
        if n_windows < 1:
            _fail(f"n_windows 必须 >= 1，实际 {n_windows}")
        if launches_per_window < 1:
            _fail(f"launches_per_window 必须 >= 1，实际 {launches_per_window}")
        self._validate_w(W)
        self._validate_x(W, x)
        self._validate_out(W, out)
        win = (ctypes.c_double * n_windows)()
        res = _capi.CqTiming()
        st = _on_device(W.device, lambda stream: self._lib.cq_native_timing(
                self._op_id(W), variant.encode(), W.data_ptr(), None,
                x.data_ptr(), out.data_ptr(), W.size(0), W.size(1), stream,
                warmup, n_windows, launches_per_window, win, ctypes.byref(res)))
        if st != _capi.CQ_OK:
            _fail(f"native_timing failed (status {st}): {_capi.last_error()}")
        return {
            "variant": variant,
            "warmup": int(warmup),
            "n_windows": int(n_windows),
            "launches_per_window": int(launches_per_window),
            "window_median_us": [float(v) for v in win],
            "median_us": res.median_us,
            "min_us": res.min_us,
            "max_us": res.max_us,
            "mean_us": res.mean_us,
            "note": NATIVE_TIMING_NOTE,
        }

    def describe(self, variant: str, W: torch.Tensor, x: torch.Tensor) -> dict:
        self._lookup(variant)
        s = _capi._string_call(self._lib.cq_describe_launch, self._op_id(W),
                               variant.encode(), W.size(0), W.size(1),
                               W.data_ptr(), x.data_ptr())
        return _capi.parse_launch_line(s)

    def contract_ok(self, W: torch.Tensor, x: torch.Tensor) -> bool:
        return bool(self._lib.cq_vec_contract_ok(self._op_id(W), W.data_ptr(),
                                                 x.data_ptr(), W.size(1)))


_EXTS: dict[str, _OpExt] = {}
_EXT_TYPES = {"int4gemv": Int4gemvExt, "qgemv": QgemvExt, "gemv": GemvExt}


def get_ext(op: str) -> _OpExt:
    """Singleton extension object for "int4gemv", "qgemv" or "gemv"."""
    if op not in _EXT_TYPES:
        raise KeyError(f"no extension for operator {op!r}")
    e = _EXTS.get(op)
    if e is None:
        e = _EXT_TYPES[op]()
        _EXTS[op] = e
    return e


# The native loop starts its host clock after it has launched the wait and
# recorded the start event, so the wait may already have run that long (a
# few microseconds on MI355X hosts) when the clock starts; a window counts as
# pre-filled only when its enqueue ended this much before the wait did.
PREFILL_MARGIN_US = 50.0


def window_prefilled(delay_us: float, host_us: float) -> bool:
    """Whether a window's on-device wait outlasted the host's enqueue of the
    window (with PREFILL_MARGIN_US to spare), so that the GPU met every
    launch of the window already queued."""
    return delay_us > 0 and host_us + PREFILL_MARGIN_US < delay_us


def prefill_delay_us(n_launches: int) -> float:
    """On-device wait to queue ahead of a window of `n_launches` launches so
    that the host has enqueued all of them before the GPU reaches the first:
    5 us per launch (host submission takes about 2.5-3.5 us per launch on
    MI355X) plus 0.5 ms, at most 1 s."""
    return float(min(1e6, 500.0 + 5.0 * n_launches))


def pool_timing(op: str, variant: str, sets: list, warmup: int,
                n_launches: int, per_kernel: bool,
                stream: Optional[torch.cuda.Stream] = None,
                burn_ms: float = 0.0, delay_us: float = 0.0) -> dict:
    """Rotating-pool launch loop in native code (cq_pool_timing).

    `sets` is a list of (W, scale, x, out) tuples of one shape ((W, x, out)
    for "gemv"), already validated by the caller.  Untimed launches run
    until both `warmup` launches and `burn_ms` of wall-clock time have
    passed; `delay_us` > 0 queues an on-device wait before the start event
    so the host enqueues the window ahead of the GPU (see
    prefill_delay_us).  Returns {"total_us": window event time,
    "host_us": host time spent enqueuing the window, "prefilled": whether
    a wait was queued and outlasted that enqueue (if not, the GPU may have
    reached the window before the host finished it), "kernel_us":
    per-launch device durations (list) or None}."""
    lib = _capi.load()
    n = len(sets)
    VP = ctypes.c_void_p * n
    if op == "gemv":
        sets = [(W, None, x, o) for (W, x, o) in sets]
    w = VP(*[s[0].data_ptr() for s in sets])
    sc = VP(*[s[1].data_ptr() for s in sets]) if op != "gemv" else None
    xs = VP(*[s[2].data_ptr() for s in sets])
    ys = VP(*[s[3].data_ptr() for s in sets])
    W0 = sets[0][0]
    N = W0.size(0)
    K = 2 * W0.size(1) if op == "int4gemv" else W0.size(1)
    op_id = _capi.OPS[op]
    if op == "gemv":
        op_id = GemvExt._op_id(W0)
    ku = (ctypes.c_float * n_launches)() if per_kernel else None
    tot = ctypes.c_double(0.0)
    host = ctypes.c_double(0.0)
    dev = W0.device
    with torch.cuda.device(dev):
        s = stream if stream is not None else torch.cuda.current_stream(dev)
        st = lib.cq_pool_timing(
            op_id, variant.encode(), w, sc, xs, ys, n, N, K,
            s.cuda_stream, warmup, float(burn_ms), float(delay_us),
            n_launches, ku, ctypes.byref(tot), ctypes.byref(host))
    if st != _capi.CQ_OK:
        _fail(f"pool_timing failed (status {st}): {_capi.last_error()}")
    return {"total_us": tot.value, "host_us": host.value,
            "prefilled": window_prefilled(delay_us, host.value),
            "kernel_us": [float(v) for v in ku] if ku is not None else None}


def read_ceiling(nbytes: int, warmup: int = 200, n_launches: int = 2000,
                 pool_bytes: int = 512 << 20, device: str = "cuda",
                 burn_ms: float = 0.0, delay_us: float = 0.0) -> dict:
    """Bandwidth ceiling of one launch reading `nbytes`: a plain streaming
    read kernel (cq_read_ceiling) over a rotating pool of distinct buffers
    totalling more than `pool_bytes` (HBM-cold), timed like pool_timing."""
    lib = _capi.load()
    nbytes = (int(nbytes) + 15) // 16 * 16
    n = max(2, pool_bytes // nbytes + 1)
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=device) for _ in range(n)]
    for b in bufs:
        b.fill_(0x5A)
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    arr = (ctypes.c_void_p * n)(*[b.data_ptr() for b in bufs])
    tot = ctypes.c_double(0.0)
    dev = bufs[0].device
    with torch.cuda.device(dev):
        s = torch.cuda.current_stream(dev)
        st = lib.cq_read_ceiling(arr, n, nbytes, sink.data_ptr(), s.cuda_stream,
                                 warmup, float(burn_ms), float(delay_us),
                                 n_launches, ctypes.byref(tot))
    if st != _capi.CQ_OK:
        _fail(f"read_ceiling failed (status {st}): {_capi.last_error()}")
    us = tot.value / n_launches
    return {"bytes": nbytes, "us_per_call": us, "GBps": nbytes / us / 1e3,
            "pool_buffers": n}


def launch_floor(grid: int, block: int, warmup: int = 200,
                 n_launches: int = 2000, device: str = "cuda",
                 burn_ms: float = 0.0, delay_us: float = 0.0) -> float:
    """µs per launch of a kernel with no memory work, `grid` workgroups of
    `block` threads, back to back on the current stream (cq_launch_floor):
    the per-dispatch cost of that launch shape in the pool-timing caliber."""
    lib = _capi.load()
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    tot = ctypes.c_double(0.0)
    with torch.cuda.device(sink.device):
        s = torch.cuda.current_stream(sink.device)
        st = lib.cq_launch_floor(int(grid), int(block), sink.data_ptr(),
                                 s.cuda_stream, warmup, float(burn_ms),
                                 float(delay_us), n_launches,
                                 ctypes.byref(tot))
    if st != _capi.CQ_OK:
        _fail(f"launch_floor failed (status {st}): {_capi.last_error()}")
    return tot.value / n_launches


# ---------------------------------------------------------------- quantizers
def _quant_launch(fn, what: str, W: torch.Tensor, q: torch.Tensor,
                  scale: torch.Tensor, rcp: bool) -> None:
    mode = _capi.CQ_SCALE_RCP if rcp else _capi.CQ_SCALE_DIV
    st = _on_device(W.device, lambda stream: fn(
        W.data_ptr(), q.data_ptr(), scale.data_ptr(), W.size(0), W.size(1),
        mode, stream))
    if st != _capi.CQ_OK:
        _fail(f"{what} failed (status {st}): {_capi.last_error()}")


def quantize_int4(W: torch.Tensor, rcp: bool = True
                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """On-device INT4 quantize + pack (cq_int4_quantize) of a CUDA fp16
    contiguous W (N, K), N, K >= 1, K % 128 == 0 (the caller checks the
    metadata).  Returns (W_packed uint8 (N, K/2), scale fp16 (N, K/128)),
    asynchronous on the current stream.  A group holding NaN/Inf gets a
    non-finite scale.  `rcp`: scale32 = amax * fl(1/7), as torch computes
    `amax / 7` for a GPU tensor; otherwise amax / 7 correctly rounded, as
    torch computes it for a CPU tensor."""
    N, K = W.shape
    wp = torch.empty((N, K // 2), dtype=torch.uint8, device=W.device)
    scale = torch.empty((N, K // 128), dtype=torch.float16, device=W.device)
    _quant_launch(_capi.load().cq_int4_quantize, "int4 quantize", W, wp, scale,
                  rcp)
    return wp, scale


def quantize_q8(W: torch.Tensor, rcp: bool = True
                ) -> tuple[torch.Tensor, torch.Tensor]:
    """On-device per-row INT8 quantize (cq_q8_quantize) of a CUDA fp16
    contiguous W (N, K), N, K >= 1.  Returns (W_q int8 (N, K), scale
    float32 (N,)), asynchronous on the current stream.  A row holding
    NaN/Inf gets a non-finite scale.  `rcp` as for quantize_int4 (with
    127)."""
    N, K = W.shape
    wq = torch.empty((N, K), dtype=torch.int8, device=W.device)
    scale = torch.empty((N,), dtype=torch.float32, device=W.device)
    _quant_launch(_capi.load().cq_q8_quantize, "int8 quantize", W, wq, scale,
                  rcp)
    return wq, scale


def quantize_vectorized(op: str, W: torch.Tensor, out: torch.Tensor) -> bool:
    """Whether the quantizer of `op` ("int4gemv" | "qgemv") takes its
    vectorized kernel for these tensors (same results either way)."""
    r = _capi.load().cq_quantize_vectorized(_capi.OPS[op], W.data_ptr(),
                                            out.data_ptr(), W.size(0), W.size(1))
    if r < 0:
        _fail(f"quantize_vectorized: {_capi.last_error()}")
    return bool(r)
