"""Build and load the gfx950 library `libcdnaqgemv.so`.

Role of the reference's `cudalab/build.py:72-114` (JIT nvcc build of a
torch extension per operator, `build("int4gemv")` returning the module),
re-designed for MI355X:

* one C-ABI shared library for both operators, compiled ahead of time with
  hipcc for `--offload-arch=gfx950` (no JIT, no torch types in the ABI), so
  the built `.so` ships with the source tree to the GPU host;
* `build(op)` returns the operator's Python extension object
  (`cudalab_amd.ext.Int4gemvExt` / `QgemvExt`) bound to the loaded library,
  with the reference module's API (`forward`, `forward_into`,
  `native_timing`, `variants`, `all_variants`, `quarantined_variants`).

Compile flags: `-O3 -std=c++20`, no fast-math (fp16 subnormals matter),
`-ffp-contract=off` (every fused multiply-add in the kernels is written out,
so the arithmetic does not depend on contraction heuristics), packed FP32
instructions disabled, and kernel arguments preloaded into scalar registers
at wave launch (`-amdgpu-kernarg-preload-count=16`).  Without the preload
every wave starts with scalar loads of its arguments and waits for them
before it can form any address; on MI355X that wait held the first weight
loads about 0.4 us after the first wave started, and preloading took the
INT4 4096x4096 streaming call from 3.79 to 3.59 us and a plain 8.7 MB read
from 2.93 to 2.58 us (queue pre-filled, same plans).  The compiler keeps a
256-byte prologue that loads the arguments the old way, for firmware that
does not preload.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB_DIR = PKG / "_lib"
LIB_NAME = "libcdnaqgemv.so"
LIB_PATH = LIB_DIR / LIB_NAME

ARCH = "gfx950"
SOURCES = ("cq_kernels.hip", "cq_quantize.hip", "cq_capi.cpp")
# the Python binding of the eager fast path (host code only, built with the
# host compiler against torch's headers; it calls the library by address)
FAST_SOURCE = "cq_pyfast.cpp"
FAST_NAME = "_cqfast"
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
)


def source_hash() -> str:
    """Stamp of what the library is built from: SHA-256 (first 16 hex
    digits) over the compile flags and the names and bytes of every file
    under cudalab_amd/csrc and include/.  Compiled into the library (its
    cq_version() string ends in "src=<stamp>") and compared on load, so a
    library built from other sources than the tree holds is refused."""
    h = hashlib.sha256()
    h.update(" ".join(HIPCC_FLAGS).encode())
    files = sorted(p for d in (CSRC, INCLUDE) for p in d.iterdir()
                   if p.is_file() and p.suffix in (".hip", ".cpp", ".h"))
    for p in files:
        h.update(b"\0" + p.name.encode() + b"\0")
        h.update(p.read_bytes())
    return h.hexdigest()[:16]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (ROCM_PATH or PATH): cannot build "
                           f"{LIB_NAME}")
    return found


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    # hipcc's host pass does not know the device-only feature flag; that
    # warning is expected and dropped from the log.
    log = "\n".join(line for line in r.stdout.splitlines()
                    if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"build failed ({r.returncode}): {' '.join(cmd)}\n"
                           f"{log}")
    if log.strip():
        print(log, file=sys.stderr)


def fast_module_path() -> Path:
    import sysconfig
    return LIB_DIR / (FAST_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


_FAST_FLAGS = ("-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
               "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1")
_FAST_LIBS = ("-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python")


def fast_abi_stamp() -> str:
    """What the fast-path module's binary interface depends on besides its
    sources: the torch version it was compiled against, torch's C++ ABI
    flag, and the compile flags and libraries of its g++ line (the include
    and library directories are left out: they name this machine's paths).
    Compiled into the module and compared on load, so a module built
    against another torch is refused rather than imported."""
    import torch
    h = hashlib.sha256(" ".join(_FAST_FLAGS + _FAST_LIBS).encode()).hexdigest()[:12]
    return (f"torch={torch.__version__};"
            f"cxx11abi={int(torch._C._GLIBCXX_USE_CXX11_ABI)};flags={h}")


def _fast_module_cmd(out: Path, stamp: str) -> list[str]:
    """g++ line of the fast-path module: torch's and Python's headers, HIP's
    host headers (for the current-stream query), linked against torch's
    libraries, which the importing process has already loaded."""
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths, library_paths
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    incs = [*include_paths(), sysconfig.get_paths()["include"],
            str(Path(rocm) / "include"), str(INCLUDE)]
    return ["g++", *_FAST_FLAGS,
            f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
            stamp, f"-DCQ_FAST_ABI=\"{fast_abi_stamp()}\"",
            *[f"-I{p}" for p in incs], str(CSRC / FAST_SOURCE),
            "-o", str(out), *[f"-L{p}" for p in library_paths()], *_FAST_LIBS]


def build_library(verbose: bool = False) -> Path:
    """Compile `libcdnaqgemv.so` and the fast-path module in-tree (always
    compiles; atomic replace).  The library is required; the fast-path
    module is best effort: if its g++ step fails the library is still
    installed, any earlier module is removed, and the operators take the
    checked path for every call (ext.py warns once)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="cq_build_", dir=LIB_DIR) as tmp:
        objs = []
        cmds = []
        stamp = f"-DCQ_SRC_HASH=\"{source_hash()}\""
        for src in SOURCES:
            obj = Path(tmp) / (Path(src).stem + ".o")
            objs.append(str(obj))
            cmds.append([cc, *HIPCC_FLAGS, stamp, f"-I{INCLUDE}", f"-I{CSRC}",
                         "-c", str(CSRC / src), "-o", str(obj)])
        fast_tmp = Path(tmp) / fast_module_path().name
        with ThreadPoolExecutor(max_workers=len(cmds) + 1) as ex:
            fast_job = ex.submit(_run, _fast_module_cmd(fast_tmp, stamp))
            for f in [ex.submit(_run, c) for c in cmds]:
                f.result()
            try:
                fast_job.result()
                os.replace(fast_tmp, fast_module_path())
            except (RuntimeError, OSError) as e:
                fast_module_path().unlink(missing_ok=True)
                print(f"warning: the eager fast-path module was not built; "
                      f"every call takes the checked path ({e})", file=sys.stderr)
        out_tmp = Path(tmp) / LIB_NAME
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs,
              "-o", str(out_tmp)])
        os.replace(out_tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def build(op: str):
    """Extension object for `op` ("int4gemv" | "qgemv" | "gemv"), bound to the built
    library.  Mirrors `cudalab/build.py:build(op)` (which returned the JIT
    module); raises if the library has not been built."""
    from . import ext
    return ext.get_ext(op)


if __name__ == "__main__":
    build_library(verbose=True)
