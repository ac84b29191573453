"""INT4 W4A16 group-wise GEMV operator adapter.

Drop-in for `cudalab/operators/int4gemv.py:100-376`: the same bench matrix,
primary target, input generators (make_w4 / make_x4), algorithmic byte
formula and suite hooks, over the gfx950 library.

    W_packed (N, K/2) uint8, scale (N, K/128) fp16, x (K,) fp16 -> y (N,) fp16
    y[n] = sum_k q[n,k] * scale[n, k/128] * x[k]   (FP32 accumulate)

Bench pools (see cudalab_amd/evaluator/bench.py for the modes): "hot" (one
set), "streaming" (HBM-cold rotating pool of > 512 MiB of distinct full
sets) and "x-rotate" (the reference's streaming: x/out rotate, W shared).
Quantization and packing run while the pool is built, outside timing.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from ..evaluator.bench import POOL_SIZE, SEED, BenchPool, cold_pool_sets
from ..int4gemv_quantize import GROUP_SIZE, quantize_w
from .base import Operator
from .gemv import make_w as _make_w_fp16, make_x as _make_x_fp16

ROOT = Path(__file__).resolve().parents[2]

# (N, K); every K is a multiple of 128
BENCH_MATRIX_INT4GEMV = [
    (1024, 4096),
    (4096, 1024),
    (4096, 4096),
    (11008, 4096),
    (4096, 11008),
]
PRIMARY_TARGET = (4096, 4096)


def make_w4(N: int, K: int, seed: int = 0, mode: str = "normal",
            scale: float = 1.0, large: float = 10.0,
            device: str = "cuda") -> tuple[torch.Tensor, torch.Tensor,
                                           torch.Tensor]:
    """Seeded fp16 W (make_w modes) quantized and packed.

    Returns (W_packed uint8 (N, K/2), scale fp16 (N, K/128), W fp16)."""
    W = _make_w_fp16(N, K, torch.float16, device=device, seed=seed,
                     mode=mode, scale=scale, large=large)
    W_packed, s = quantize_w(W)
    return W_packed, s, W


def make_x4(K: int, seed: int = 0, mode: str = "normal", large: float = 10.0,
            device: str = "cuda") -> torch.Tensor:
    return _make_x_fp16(K, torch.float16, device=device, seed=seed,
                        mode=mode, large=large)


def int4_bytes(N: int, K: int) -> int:
    """Algorithmic bytes of one call: W_packed + scale + x + y."""
    return N * K // 2 + N * (K // GROUP_SIZE) * 2 + 2 * K + 2 * N


def device_random_set(N: int, K: int, seed: int, device: str = "cuda",
                      w_std: float = 0.02):
    """One (W_packed, scale, x, out) set drawn with the device generator:
    W ~ N(0, w_std) fp16 quantized on the device, x ~ N(0, 1) fp16.  Used
    to fill large timing pools quickly (values do not affect timing)."""
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    W = (torch.randn(N, K, generator=g, device=device) * w_std).half()
    W_packed, s = quantize_w(W)
    del W
    x = torch.randn(K, generator=g, device=device).half()
    out = torch.empty(N, dtype=torch.float16, device=device)
    return W_packed, s, x, out


class Int4gemvOperator(Operator):
    name = "int4gemv"
    dtypes = ("float16",)
    bench_shapes = BENCH_MATRIX_INT4GEMV
    primary_target = PRIMARY_TARGET
    kernel_regex = "int4gemv"
    ncu_kernel_regex = "int4gemv"
    profiles_dir = ROOT / "profiles"
    bench_dir = ROOT / "benchmarks" / "int4gemv"
    experiments_dir = ROOT / "experiments" / "int4gemv"

    def build(self):
        from ..build import build
        return build("int4gemv")

    def make_bench_pool(self, M: int, K: int, dtype: torch.dtype, mode: str,
                        seed: int = SEED, pool_size: int = POOL_SIZE
                        ) -> BenchPool:
        """Preallocate every tensor a timed launch touches.  (M, K) is
        (N, K)."""
        N = M
        if dtype != torch.float16:
            raise NotImplementedError(f"int4gemv takes fp16 activations only, "
                                      f"got {dtype}")
        if K % GROUP_SIZE != 0:
            raise NotImplementedError(f"int4gemv needs K % 128 == 0, got K={K}")
        dev = "cuda"
        wp_bytes = N * K // 2
        scale_bytes = N * (K // GROUP_SIZE) * 2
        set_bytes = int4_bytes(N, K)
        if mode == "streaming":
            n = max(pool_size, cold_pool_sets(set_bytes))
            sets = [device_random_set(N, K, seed + 100000 + i, dev)
                    for i in range(n)]
            xs = [s[2] for s in sets]
            outs = [s[3] for s in sets]

            def launch(ext, variant, i):
                W, s, x, o = sets[i]
                ext.forward_into(variant, W, s, x, o)

            return BenchPool(xs=xs, outs=outs, pool_size=n,
                             working_set_bytes=n * set_bytes, element_size=2,
                             mode=mode, launch=launch, sets=sets,
                             op="int4gemv", shared_bytes=0,
                             pool_extra={"hbm_cold": True,
                                         "distinct_sets": n,
                                         "set_bytes": set_bytes,
                                         "pool_bytes": n * set_bytes})
        n = 1 if mode == "hot" else pool_size
        W_packed, scale, _ = make_w4(N, K, seed=seed + 100000, device=dev)
        xs = [make_x4(K, seed=seed + i, device=dev) for i in range(n)]
        outs = [torch.empty(N, dtype=torch.float16, device=dev) for _ in xs]
        shared = {"W_packed": W_packed, "scale": scale}

        def launch(ext, variant, i):
            ext.forward_into(variant, shared["W_packed"], shared["scale"],
                             xs[i], outs[i])

        return BenchPool(xs=xs, outs=outs, pool_size=n,
                         working_set_bytes=n * 2 * (K + N), element_size=2,
                         mode=mode, launch=launch, shared=shared,
                         sets=[(W_packed, scale, xs[i], outs[i]) for i in range(n)],
                         op="int4gemv", shared_bytes=wp_bytes + scale_bytes,
                         pool_extra={"hbm_cold": False,
                                     "weights_resident": True,
                                     "W_packed_bytes": wp_bytes,
                                     "scale_bytes": scale_bytes})

    def algorithmic_bytes(self, M: int, K: int, element_size: int = 2) -> int:
        """N*K/2 (W_packed) + N*K/128*2 (scale) + 2K (x) + 2N (y)."""
        return int4_bytes(M, K)

    def profile_driver_source(self, variant: str, M: int, K: int) -> str:
        return f"""
import sys
sys.path.insert(0, {str(ROOT)!r})
import torch
from cudalab_amd.build import build
from cudalab_amd.operators.int4gemv import make_w4, make_x4

ext = build("int4gemv")
W_packed, scale, _W = make_w4({M}, {K}, seed=1234)
x = make_x4({K}, seed=1234)
out = torch.empty({M}, dtype=torch.float16, device="cuda")
for _ in range(6):
    ext.forward_into("{variant}", W_packed, scale, x, out)
torch.cuda.synchronize()
print("profile driver done")
"""

    def experiment_prefix(self) -> str:
        return "INT4GEMV"

    def run_correctness(self, ext, variant: str,
                        out_dir: Path | None = None) -> dict:
        from ..int4gemv_correctness import (run_fidelity_suite, run_suite,
                                            save_fidelity, save_results,
                                            summarize)
        out_dir = Path(out_dir or self.experiments_dir / "correctness")
        out_dir.mkdir(parents=True, exist_ok=True)
        results = run_suite(variant, ext)
        saved = save_results(results, out_dir / f"{variant}.json")
        s = summarize(results)
        fid_path = out_dir / "quantization_fidelity.json"
        if fid_path.exists():
            fid_summary = json.loads(fid_path.read_text()).get("summary")
        else:
            fid = run_fidelity_suite()
            save_fidelity(fid, fid_path)
            fid_summary = fid["summary"]
        return {"all_pass": bool(s["all_pass"]), "summary": s,
                "saved": str(saved),
                "quantization_fidelity": {"saved": str(fid_path),
                                          "summary": fid_summary}}

    def run_negative(self, ext, variant: str | None = None,
                     out_dir: Path | None = None) -> dict:
        from ..int4gemv_negative import run_negative_suite
        v = variant or "int4gemv_baseline"
        out_dir = Path(out_dir or self.experiments_dir / "correctness")
        out_dir.mkdir(parents=True, exist_ok=True)
        name = ("invalid_inputs.json" if v == "int4gemv_baseline"
                else f"invalid_inputs_{v}.json")
        return run_negative_suite(ext, out_path=out_dir / name, variant=v)

    def pytorch_ref_latency(self, M: int, K: int, dtype: torch.dtype,
                            iters: int = 200, batch: int = 32) -> dict:
        """Framework context: torch.mv on the unquantized fp16 W (hipBLAS);
        PyTorch has no W4A16 GEMV op."""
        from ..evaluator.bench import time_call
        if dtype not in (torch.float16, "float16"):
            return {"available": True, "error": "fp16 activations only"}
        _wp, _s, W = make_w4(M, K, seed=SEED)
        x = make_x4(K, seed=SEED)
        t = time_call(lambda: torch.mv(W, x), warmup=100, iters=iters,
                      batch=batch)
        return {"available": True, "api": "torch.mv(W_fp16, x_fp16)", **t,
                "note": "framework context only (unquantized fp16 GEMV)"}


int4gemv = Int4gemvOperator()
