"""Seeded input generators shared by the GEMV operators, and the FP16/FP32
GEMV operator adapter (below).

Drop-in for `make_w` / `make_x` of `cudalab/operators/gemv.py:106-190`
(same modes and arguments).  Difference by design: the random stream comes
from a CPU `torch.Generator` and the tensor is then moved to `device`, so
the same seed gives the same values on every host (the reference drew on
the GPU generator, whose stream is tied to the device).

Modes:
  normal      N(0, scale)
  zeros       all zero
  tiny        N(0, 1e-4)   (many fp16 subnormals in x)
  large       N(0, large)
  mixed_sign  W: |N(0,1)| * (-1)^(i+j);  x: |N(0,1)| * independent random
              signs, so that W[i,j]*x[j] has independent signs along a row
              (real cancellation).
"""
from __future__ import annotations

import torch

MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    return g


def make_w(N: int, K: int, dtype: torch.dtype, device: str = "cuda",
           seed: int = 0, mode: str = "normal", scale: float = 1.0,
           large: float = 10.0) -> torch.Tensor:
    g = _gen(seed)
    if mode == "normal":
        w = torch.randn(N, K, generator=g) * scale
    elif mode == "zeros":
        w = torch.zeros(N, K)
    elif mode == "tiny":
        w = torch.randn(N, K, generator=g) * 1e-4
    elif mode == "large":
        w = torch.randn(N, K, generator=g) * large
    elif mode == "mixed_sign":
        mag = torch.randn(N, K, generator=g).abs()
        parity = (torch.arange(N).unsqueeze(1) + torch.arange(K).unsqueeze(0)) % 2
        w = torch.where(parity == 0, mag, -mag)
    else:
        raise ValueError(f"unknown input mode: {mode!r}")
    return w.to(dtype).contiguous().to(device)


def make_x(K: int, dtype: torch.dtype, device: str = "cuda", seed: int = 0,
           mode: str = "normal", scale: float = 1.0,
           large: float = 10.0) -> torch.Tensor:
    g = _gen(seed)
    if mode == "normal":
        x = torch.randn(K, generator=g) * scale
    elif mode == "zeros":
        x = torch.zeros(K)
    elif mode == "tiny":
        x = torch.randn(K, generator=g) * 1e-4
    elif mode == "large":
        x = torch.randn(K, generator=g) * large
    elif mode == "mixed_sign":
        mag = torch.randn(K, generator=g).abs()
        bits = torch.randint(0, 2, (K,), generator=g)
        x = torch.where(bits == 0, mag, -mag)
    else:
        raise ValueError(f"unknown input mode: {mode!r}")
    return x.to(dtype).contiguous().to(device)


# --------------------------------------------------------------------------
# FP16/FP32 GEMV operator adapter (the reference's third generation)
#
# Drop-in for `GemvOperator` of cudalab/operators/gemv.py:88-340: the same
# bench matrix, reference formulation (gemv_ref), byte formula and suite
# hooks, over the gfx950 library.
#     W (N, K), x (K,) -> y (N,), all fp16 or all fp32
#     y[n] = sum_k W[n,k] * x[k]   (FP32 accumulate, one cast)

from pathlib import Path as _Path                             # noqa: E402

from ..evaluator.bench import (POOL_SIZE, SEED, BenchPool,     # noqa: E402
                               cold_pool_sets)
from .base import Operator                                     # noqa: E402

_ROOT = _Path(__file__).resolve().parents[2]

BENCH_MATRIX_GEMV = [
    (1024, 4096),
    (4096, 1024),
    (4096, 4096),
    (11008, 4096),
    (4096, 11008),
]
PRIMARY_TARGET = (4096, 4096)


def gemv_ref(W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """The reference formulation: FP32 matvec, cast back to W's dtype
    (cudalab/operators/gemv.py:192-200)."""
    if W.dim() != 2:
        raise ValueError(f"expected a 2-D W (N, K), got {W.dim()}-D")
    if x.dim() != 1:
        raise ValueError(f"expected a 1-D x (K,), got {x.dim()}-D")
    if W.dtype == torch.float16:
        return torch.mv(W.float(), x.float()).to(torch.float16)
    return torch.mv(W, x)


def gemv_bytes(N: int, K: int, element_size: int) -> int:
    """Algorithmic bytes of one call: W + x + y."""
    return (N * K + K + N) * element_size


def device_random_set(N: int, K: int, seed: int, dtype=torch.float16,
                      device: str = "cuda"):
    """One (W, x, out) set drawn with the device generator (timing pools)."""
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    W = (torch.randn(N, K, generator=g, device=device) * 0.02).to(dtype)
    x = torch.randn(K, generator=g, device=device).to(dtype)
    out = torch.empty(N, dtype=dtype, device=device)
    return W, x, out


class GemvOperator(Operator):
    name = "gemv"
    dtypes = ("float16", "float32")
    bench_shapes = BENCH_MATRIX_GEMV
    primary_target = PRIMARY_TARGET
    kernel_regex = "gemv_"
    ncu_kernel_regex = "gemv_"
    profiles_dir = _ROOT / "profiles"
    bench_dir = _ROOT / "benchmarks" / "gemv"
    experiments_dir = _ROOT / "experiments" / "gemv"

    def build(self):
        from ..build import build
        return build("gemv")

    def make_bench_pool(self, M: int, K: int, dtype: torch.dtype, mode: str,
                        seed: int = SEED, pool_size: int = POOL_SIZE
                        ) -> BenchPool:
        """Preallocate every tensor a timed launch touches.  (M, K) is
        (N, K)."""
        N = M
        es = torch.tensor([], dtype=dtype).element_size()
        dev = "cuda"
        set_bytes = gemv_bytes(N, K, es)
        if mode == "streaming":
            n = max(pool_size, cold_pool_sets(set_bytes))
            sets = [device_random_set(N, K, seed + 100000 + i, dtype, dev)
                    for i in range(n)]

            def launch(ext, variant, i):
                W, x, o = sets[i]
                ext.forward_into(variant, W, x, o)

            return BenchPool(xs=[s[1] for s in sets], outs=[s[2] for s in sets],
                             pool_size=n, working_set_bytes=n * set_bytes,
                             element_size=es, mode=mode, launch=launch,
                             sets=sets, op="gemv", shared_bytes=0,
                             pool_extra={"hbm_cold": True, "distinct_sets": n,
                                         "set_bytes": set_bytes,
                                         "pool_bytes": n * set_bytes})
        n = 1 if mode == "hot" else pool_size
        W = make_w(N, K, dtype, device=dev, seed=seed + 100000)
        xs = [make_x(K, dtype, device=dev, seed=seed + i) for i in range(n)]
        outs = [torch.empty(N, dtype=dtype, device=dev) for _ in xs]
        shared = {"W": W}

        def launch(ext, variant, i):
            ext.forward_into(variant, shared["W"], xs[i], outs[i])

        return BenchPool(xs=xs, outs=outs, pool_size=n,
                         working_set_bytes=n * es * (K + N), element_size=es,
                         mode=mode, launch=launch, shared=shared,
                         sets=[(W, xs[i], outs[i]) for i in range(n)],
                         op="gemv", shared_bytes=N * K * es,
                         pool_extra={"hbm_cold": False, "weights_resident": True,
                                     "W_bytes": N * K * es})

    def algorithmic_bytes(self, M: int, K: int, element_size: int = 2) -> int:
        """(N*K + K + N) * element size (cudalab/operators/gemv.py:283-289)."""
        return gemv_bytes(M, K, element_size)

    def profile_driver_source(self, variant: str, M: int, K: int) -> str:
        return f"""
import sys
sys.path.insert(0, {str(_ROOT)!r})
import torch
from cudalab_amd.build import build
from cudalab_amd.operators.gemv import make_w, make_x

ext = build("gemv")
W = make_w({M}, {K}, torch.float16, seed=1234)
x = make_x({K}, torch.float16, seed=1235)
out = torch.empty({M}, dtype=torch.float16, device="cuda")
for _ in range(6):
    ext.forward_into("{variant}", W, x, out)
torch.cuda.synchronize()
print("profile driver done")
"""

    def experiment_prefix(self) -> str:
        return "GEMV"

    def run_correctness(self, ext, variant: str, out_dir=None) -> dict:
        from ..gemv_correctness import run_suite, save_results, summarize
        out_dir = _Path(out_dir or self.experiments_dir / "correctness")
        out_dir.mkdir(parents=True, exist_ok=True)
        results = run_suite(variant, ext)
        saved = save_results(results, out_dir / f"{variant}.json")
        s = summarize(results)
        return {"all_pass": bool(s["all_pass"]), "summary": s,
                "saved": str(saved)}

    def run_negative(self, ext, variant: str | None = None,
                     out_dir=None) -> dict:
        from ..gemv_negative import run_negative_suite
        v = variant or "gemv_baseline"
        out_dir = _Path(out_dir or self.experiments_dir / "correctness")
        out_dir.mkdir(parents=True, exist_ok=True)
        name = ("invalid_inputs.json" if v == "gemv_baseline"
                else f"invalid_inputs_{v}.json")
        return run_negative_suite(ext, out_path=out_dir / name, variant=v)

    def pytorch_ref_latency(self, M: int, K: int, dtype: torch.dtype,
                            iters: int = 200, batch: int = 32) -> dict:
        """Framework context: torch.mv (hipBLAS) on the same shape."""
        from ..evaluator.bench import time_call
        W = make_w(M, K, dtype, seed=SEED)
        x = make_x(K, dtype, seed=SEED + 1)
        t = time_call(lambda: torch.mv(W, x), warmup=100, iters=iters,
                      batch=batch)
        return {"available": True, "api": "torch.mv(W, x)", **t}


gemv = GemvOperator()
