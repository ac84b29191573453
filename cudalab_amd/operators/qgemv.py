"""INT8 W8A16 per-row GEMV operator adapter.

Drop-in for `cudalab/operators/qgemv.py:87-340`.

    W_q (N, K) int8, scale (N,) float32, x (K,) fp16 -> y (N,) fp16
    y[n] = scale[n] * sum_k W_q[n,k] * x[k]   (FP32 accumulate)
"""
from __future__ import annotations

from pathlib import Path

import torch

from ..evaluator.bench import POOL_SIZE, SEED, BenchPool, cold_pool_sets
from ..qgemv_quantize import quantize_w
from .base import Operator
from .gemv import make_w as _make_w_fp16, make_x as _make_x_fp16

ROOT = Path(__file__).resolve().parents[2]

BENCH_MATRIX_QGEMV = [
    (1024, 4096),
    (4096, 1024),
    (4096, 4096),
    (11008, 4096),
    (4096, 11008),
]
PRIMARY_TARGET = (4096, 4096)


def make_w_q(N: int, K: int, seed: int = 0, mode: str = "normal",
             scale: float = 1.0, large: float = 10.0,
             device: str = "cuda") -> tuple[torch.Tensor, torch.Tensor,
                                            torch.Tensor]:
    """Seeded fp16 W quantized per row: (W_q int8, scale fp32 (N,), W)."""
    W = _make_w_fp16(N, K, torch.float16, device=device, seed=seed,
                     mode=mode, scale=scale, large=large)
    W_q, s = quantize_w(W)
    return W_q, s, W


def make_x_q(K: int, seed: int = 0, mode: str = "normal", large: float = 10.0,
             device: str = "cuda") -> torch.Tensor:
    return _make_x_fp16(K, torch.float16, device=device, seed=seed,
                        mode=mode, large=large)


def q8_bytes(N: int, K: int) -> int:
    """Algorithmic bytes of one call: W_q + x + scale (fp32) + y."""
    return N * K + 2 * K + 4 * N + 2 * N


def device_random_set(N: int, K: int, seed: int, device: str = "cuda",
                      w_std: float = 0.02):
    """One (W_q, scale, x, out) set drawn with the device generator."""
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    W = (torch.randn(N, K, generator=g, device=device) * w_std).half()
    W_q, s = quantize_w(W)
    del W
    x = torch.randn(K, generator=g, device=device).half()
    out = torch.empty(N, dtype=torch.float16, device=device)
    return W_q, s, x, out


class QgemvOperator(Operator):
    name = "qgemv"
    dtypes = ("float16",)
    bench_shapes = BENCH_MATRIX_QGEMV
    primary_target = PRIMARY_TARGET
    kernel_regex = "qgemv"
    ncu_kernel_regex = "qgemv"
    profiles_dir = ROOT / "profiles"
    bench_dir = ROOT / "benchmarks" / "qgemv"
    experiments_dir = ROOT / "experiments" / "qgemv"

    def build(self):
        from ..build import build
        return build("qgemv")

    def make_bench_pool(self, M: int, K: int, dtype: torch.dtype, mode: str,
                        seed: int = SEED, pool_size: int = POOL_SIZE
                        ) -> BenchPool:
        N = M
        if dtype != torch.float16:
            raise NotImplementedError(f"qgemv takes fp16 activations only, "
                                      f"got {dtype}")
        dev = "cuda"
        set_bytes = q8_bytes(N, K)
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
                             mode=mode, launch=launch, sets=sets, op="qgemv",
                             pool_extra={"hbm_cold": True, "distinct_sets": n,
                                         "set_bytes": set_bytes,
                                         "pool_bytes": n * set_bytes})
        n = 1 if mode == "hot" else pool_size
        W_q, scale, _ = make_w_q(N, K, seed=seed + 100000, device=dev)
        xs = [make_x_q(K, seed=seed + i, device=dev) for i in range(n)]
        outs = [torch.empty(N, dtype=torch.float16, device=dev) for _ in xs]
        shared = {"W_q": W_q, "scale": scale}

        def launch(ext, variant, i):
            ext.forward_into(variant, shared["W_q"], shared["scale"], xs[i],
                             outs[i])

        return BenchPool(xs=xs, outs=outs, pool_size=n,
                         working_set_bytes=n * 2 * (K + N), element_size=2,
                         mode=mode, launch=launch, shared=shared,
                         sets=[(W_q, scale, xs[i], outs[i]) for i in range(n)],
                         op="qgemv", shared_bytes=N * K + 4 * N,
                         pool_extra={"hbm_cold": False,
                                     "weights_resident": True})

    def algorithmic_bytes(self, M: int, K: int, element_size: int = 2) -> int:
        """N*K (W_q) + 2K (x) + 4N (scale) + 2N (y)."""
        return q8_bytes(M, K)

    def profile_driver_source(self, variant: str, M: int, K: int) -> str:
        return f"""
import sys
sys.path.insert(0, {str(ROOT)!r})
import torch
from cudalab_amd.build import build
from cudalab_amd.operators.qgemv import make_w_q, make_x_q

ext = build("qgemv")
W_q, scale, _W = make_w_q({M}, {K}, seed=1234)
x = make_x_q({K}, seed=1234)
out = torch.empty({M}, dtype=torch.float16, device="cuda")
for _ in range(6):
    ext.forward_into("{variant}", W_q, scale, x, out)
torch.cuda.synchronize()
print("profile driver done")
"""

    def experiment_prefix(self) -> str:
        return "QGEMV"

    def run_correctness(self, ext, variant: str,
                        out_dir: Path | None = None) -> dict:
        from ..qgemv_correctness import (run_fidelity_suite, run_suite,
                                         save_fidelity, save_results,
                                         summarize)
        out_dir = Path(out_dir or self.experiments_dir / "correctness")
        out_dir.mkdir(parents=True, exist_ok=True)
        results = run_suite(variant, ext)
        saved = save_results(results, out_dir / f"{variant}.json")
        s = summarize(results)
        fid = run_fidelity_suite()
        fid_saved = save_fidelity(fid, out_dir / "quantization_fidelity.json")
        return {"all_pass": bool(s["all_pass"]), "summary": s,
                "saved": str(saved),
                "quantization_fidelity": {"saved": str(fid_saved),
                                          "summary": fid["summary"]}}

    def run_negative(self, ext, variant: str | None = None,
                     out_dir: Path | None = None) -> dict:
        from ..qgemv_negative import run_negative_suite
        v = variant or "qgemv_baseline"
        out_dir = Path(out_dir or self.experiments_dir / "correctness")
        out_dir.mkdir(parents=True, exist_ok=True)
        name = ("invalid_inputs.json" if v == "qgemv_baseline"
                else f"invalid_inputs_{v}.json")
        return run_negative_suite(ext, out_path=out_dir / name, variant=v)

    def pytorch_ref_latency(self, M: int, K: int, dtype: torch.dtype,
                            iters: int = 200, batch: int = 32) -> dict:
        from ..evaluator.bench import time_call
        if dtype not in (torch.float16, "float16"):
            return {"available": True, "error": "fp16 activations only"}
        _wq, _s, W = make_w_q(M, K, seed=SEED)
        x = make_x_q(K, seed=SEED)
        t = time_call(lambda: torch.mv(W, x), warmup=100, iters=iters,
                      batch=batch)
        return {"available": True, "api": "torch.mv(W_fp16, x_fp16)", **t,
                "note": "framework context only (unquantized fp16 GEMV)"}


qgemv = QgemvOperator()
