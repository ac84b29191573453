"""Throughput of the on-device quantizers against the torch formulation
they replace (cudalab/int4gemv_quantize.py:61-114, cudalab/qgemv_quantize.py:
33-64, which the reference runs as a sequence of torch ops), on one GPU.

Per shape and quantizer:
  hip_us     one cq_int4_quantize / cq_q8_quantize launch, from a HIP graph
             of `launches` back-to-back launches over a rotating pool of
             distinct weights (> 512 MiB, HBM-cold), replayed between two
             events: device time per launch without host launch overhead
  torch_us   quantize_w_torch on the same GPU (the reference's code path),
             Python loop between two events, one resident W
  GBps       algorithmic bytes / hip_us: read 2NK (fp16 W), write NK/2 +
             N(K/128)*2 (INT4) or NK + 4N (INT8)

Usage: python -m cudalab_amd.evaluator.quantize_bench [--launches 200]
       [--json FILE]
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from .. import _capi
from .bench import cold_pool_sets

HBM_PEAK_GBS = 8000.0
SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]
OPS = ("int4", "int8")


def algorithmic_bytes(op: str, N: int, K: int) -> int:
    if op == "int4":
        return 2 * N * K + N * K // 2 + N * (K // 128) * 2
    return 2 * N * K + N * K + 4 * N


def _outputs(op: str, N: int, K: int, device):
    if op == "int4":
        return (torch.empty(N, K // 2, dtype=torch.uint8, device=device),
                torch.empty(N, K // 128, dtype=torch.float16, device=device))
    return (torch.empty(N, K, dtype=torch.int8, device=device),
            torch.empty(N, dtype=torch.float32, device=device))


def make_pool(op: str, N: int, K: int, seed: int = 99, device: str = "cuda"):
    """Distinct fp16 W ~ N(0, 0.02) with preallocated outputs, more than
    512 MiB in all."""
    n = cold_pool_sets(algorithmic_bytes(op, N, K))
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pool = []
    for _ in range(n):
        W = (torch.randn(N, K, generator=g, device=device) * 0.02).half()
        pool.append((W, *_outputs(op, N, K, device)))
    return pool


def hip_us(op: str, pool, launches: int = 200, warmup_replays: int = 2) -> float:
    """Device µs per launch: `launches` launches over the pool captured in
    one HIP graph, replayed between two events."""
    lib = _capi.load()
    fn = lib.cq_int4_quantize if op == "int4" else lib.cq_q8_quantize
    N, K = pool[0][0].shape
    args = [(W.data_ptr(), q.data_ptr(), s.data_ptr()) for (W, q, s) in pool]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=side):
        st = side.cuda_stream
        for i in range(launches):
            w, q, s = args[i % len(args)]
            rc = fn(w, q, s, N, K, _capi.CQ_SCALE_RCP, st)
            if rc != _capi.CQ_OK:
                raise RuntimeError(f"quantize launch failed: {_capi.last_error()}")
    for _ in range(warmup_replays):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / launches


def torch_us(op: str, W: torch.Tensor, iters: int = 20) -> float:
    if op == "int4":
        from ..int4gemv_quantize import quantize_w_torch
    else:
        from ..qgemv_quantize import quantize_w_torch
    for _ in range(3):
        quantize_w_torch(W)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        quantize_w_torch(W)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / iters


def run(ops=OPS, shapes=SHAPES, launches: int = 200) -> list[dict]:
    out = []
    for op in ops:
        for (N, K) in shapes:
            print(f"quantize_bench: {op} N={N} K={K}", file=sys.stderr, flush=True)
            pool = make_pool(op, N, K)
            us = hip_us(op, pool, launches)
            tus = torch_us(op, pool[0][0])
            nb = algorithmic_bytes(op, N, K)
            out.append({"op": op, "N": N, "K": K, "pool_sets": len(pool),
                        "bytes_per_call": nb, "hip_us": round(us, 3),
                        "GBps": round(nb / us / 1e3, 1),
                        "frac_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
                        "torch_us": round(tus, 2),
                        "speedup_vs_torch": round(tus / us, 1)})
            del pool
            torch.cuda.empty_cache()
    return out


def table(recs: list[dict]) -> str:
    lines = [f"{'op':<5} {'N':>6} {'K':>6} {'hip us':>8} {'GB/s':>7} {'%peak':>6} "
             f"{'torch us':>9} {'x torch':>8}"]
    for r in recs:
        lines.append(f"{r['op']:<5} {r['N']:>6} {r['K']:>6} {r['hip_us']:>8.2f} "
                     f"{r['GBps']:>7.0f} {100 * r['frac_peak']:>5.1f}% "
                     f"{r['torch_us']:>9.1f} {r['speedup_vs_torch']:>8.1f}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--launches", type=int, default=200)
    ap.add_argument("--json", default=None)
    a = ap.parse_args(argv)
    print(f"library: {_capi.version()}", flush=True)   # the build that ran
    if not torch.cuda.is_available():
        print("quantize_bench: no GPU visible", file=sys.stderr)
        return 1
    recs = run(launches=a.launches)
    print(table(recs), flush=True)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(recs, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
