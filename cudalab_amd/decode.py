"""Decode-step driver: the seven weight projections of every layer of a
Llama-shaped model (7B or 70B), back to back on one GPU, through the INT4
(or INT8) GEMV path.  No counterpart in the reference (it excludes model
integration: README.md:34-35); this restates the "back-to-back Llama-7B
decode projections" workload of the benchmark configuration.

Per layer, hidden H, intermediate I and k/v width KV (KV = H without
grouped-query attention; Llama-70B: H = 8192, I = 28672, KV = 1024):
  q         H -> H   from the layer input       (q, k, v independent:
  k, v      H -> KV  from the layer input        one group)
  o         H -> H   from v                     (a single-token context makes
                                                 attention the identity on v;
                                                 with KV < H each kv head's v
                                                 is repeated for its H/KV
                                                 query heads, one small copy)
  gate, up  H -> I   from o                     (independent: one group)
  down      I -> H   from up                    (feeds the next layer)
Norms, attention over a longer context, the residual adds and the SwiGLU
product are outside the GEMV path and are not modelled; the data
dependencies between projections follow the layer's order.  At 70B the
down projection (K = 28672) runs the K-tiled kernel.

Weights are random-init: W ~ N(0, 1/K) in fp16 (so activations stay O(1)
through all layers), quantized with the path's own quantizers on the
device.  Three ways to run one decode step over all layers:
  sequential  one launch per projection (7 per layer)
  grouped     q/k/v and gate/up as grouped launches (4 per layer)
  graph       the grouped step captured once in a HIP graph and replayed
All three produce bit-identical outputs.

Usage: python -m cudalab_amd.decode [--model 7b|70b] [--layers N]
       [--op int4gemv|qgemv] [--steps 20] [--warmup 3]
       [--modes sequential,grouped,graph]
       python -m cudalab_amd.decode --stress [--op int4gemv|qgemv] [--steps 20]

--stress times the decode stress sequence instead, Llama-7B projection shapes
(N, K) = (11008, 4096), (4096, 11008), then four (4096, 4096), back to back,
over an HBM-cold pool of distinct weights, replayed from a HIP graph and
run eager.
"""
from __future__ import annotations

import argparse
import json
import sys
from dataclasses import dataclass, field

import torch

from .build import build

HIDDEN = 4096
INTER = 11008
LAYERS = 32
HEAD_DIM = 128
# Llama-shaped presets: hidden, intermediate, k/v width, layers
MODELS = {"7b": dict(hidden=4096, inter=11008, kv=4096, layers=32),
          "70b": dict(hidden=8192, inter=28672, kv=1024, layers=80)}
VARIANT = {"int4gemv": "int4gemv_cdna4", "qgemv": "qgemv_cdna4"}


def projections(hidden: int, inter: int, kv: int):
    """(name, N, K) of one layer's seven projections."""
    return (("q", hidden, hidden), ("k", kv, hidden), ("v", kv, hidden),
            ("o", hidden, hidden), ("gate", inter, hidden), ("up", inter, hidden),
            ("down", hidden, inter))


PROJ = projections(HIDDEN, INTER, HIDDEN)


def _quantize(op: str, W: torch.Tensor):
    if op == "int4gemv":
        from .int4gemv_quantize import quantize_w
    else:
        from .qgemv_quantize import quantize_w
    return quantize_w(W)


def proj_bytes(op: str, N: int, K: int) -> int:
    if op == "int4gemv":
        from .operators.int4gemv import int4_bytes
        return int4_bytes(N, K)
    from .operators.qgemv import q8_bytes
    return q8_bytes(N, K)


@dataclass
class Layer:
    w: dict = field(default_factory=dict)      # name -> (W, scale)
    out: dict = field(default_factory=dict)    # name -> fp16 output buffer


class DecodeModel:
    """Quantized projection weights and activation buffers of `layers`
    layers, all resident on `device`."""

    def __init__(self, op: str = "int4gemv", layers: int = LAYERS,
                 seed: int = 7, device: str = "cuda",
                 hidden: int = HIDDEN, inter: int = INTER,
                 kv: int | None = None):
        self.op = op
        self.ext = build(op)
        self.variant = VARIANT[op]
        kv = hidden if kv is None else kv
        if hidden % kv or kv % HEAD_DIM:
            raise ValueError(f"k/v width {kv} must divide hidden {hidden} and be a "
                             f"multiple of the head size {HEAD_DIM}")
        self.hidden, self.inter, self.kv = hidden, inter, kv
        self.proj = projections(hidden, inter, kv)
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.layers: list[Layer] = []
        for _ in range(layers):
            L = Layer()
            for name, N, K in self.proj:
                W = (torch.randn(N, K, generator=g, device=device)
                     / K ** 0.5).half()
                L.w[name] = _quantize(op, W)
                L.out[name] = torch.empty(N, dtype=torch.float16, device=device)
                del W
            # o's input: v itself, or v repeated per query head group
            L.out["o_in"] = (L.out["v"] if kv == hidden else
                             torch.empty(hidden, dtype=torch.float16, device=device))
            self.layers.append(L)
        self.x0 = (torch.randn(hidden, generator=g, device=device)).half()
        self.bytes_per_step = layers * sum(proj_bytes(op, N, K)
                                           for _, N, K in self.proj)

    # -- one decode step over all layers ---------------------------------
    def _one(self, L: Layer, name: str, x: torch.Tensor):
        W, s = L.w[name]
        self.ext.forward_into(self.variant, W, s, x, L.out[name])

    def _group(self, L: Layer, names, x: torch.Tensor):
        self.ext.forward_grouped(self.variant, [(L.w[n][0], L.w[n][1], x, L.out[n])
                                                for n in names])

    def _attend(self, L: Layer) -> torch.Tensor:
        """Attention over a single-token context: each query head gets its
        kv head's v (a copy when k/v are narrower than the hidden size)."""
        if self.kv == self.hidden:
            return L.out["v"]
        kvh, rep = self.kv // HEAD_DIM, self.hidden // self.kv
        L.out["o_in"].view(kvh, rep, HEAD_DIM).copy_(
            L.out["v"].view(kvh, 1, HEAD_DIM).expand(kvh, rep, HEAD_DIM))
        return L.out["o_in"]

    def step_sequential(self) -> torch.Tensor:
        x = self.x0
        for L in self.layers:
            for n in ("q", "k", "v"):
                self._one(L, n, x)
            self._one(L, "o", self._attend(L))
            for n in ("gate", "up"):
                self._one(L, n, L.out["o"])
            self._one(L, "down", L.out["up"])
            x = L.out["down"]
        return x

    def step_grouped(self) -> torch.Tensor:
        x = self.x0
        for L in self.layers:
            self._group(L, ("q", "k", "v"), x)
            self._one(L, "o", self._attend(L))
            self._group(L, ("gate", "up"), L.out["o"])
            self._one(L, "down", L.out["up"])
            x = L.out["down"]
        return x

    def capture(self) -> torch.cuda.CUDAGraph:
        """The grouped step recorded once into a HIP graph (on a side stream,
        after one eager warm-up step)."""
        self.step_grouped()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.graph(g, stream=side):
            self.step_grouped()
        torch.cuda.synchronize()
        return g

    def outputs(self) -> list[torch.Tensor]:
        return [L.out[n].clone() for L in self.layers for n, _, _ in self.proj]

    def layer_bytes(self) -> int:
        return self.bytes_per_step // len(self.layers)


def time_steps(fn, steps: int, warmup: int) -> float:
    """Mean µs per call of `fn` over `steps` calls between two events, after
    `warmup` untimed calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


MODES = ("sequential", "grouped", "graph")

# The decode stress sequence: Llama-7B projection shapes back to back, the
# MLP pair and then four 4096^2 projections (each launch's input is its own x).
STRESS_SHAPES = ((11008, 4096), (4096, 11008), (4096, 4096), (4096, 4096),
                 (4096, 4096), (4096, 4096))
STRESS_POOL_BYTES = 512 << 20


def stress(op: str = "int4gemv", replays: int = 20, warmup: int = 3,
           pool_bytes: int = STRESS_POOL_BYTES) -> dict:
    """The stress sequence over HBM-cold weights: enough distinct copies of
    the six (W, scale, x, out) sets that together they exceed `pool_bytes`
    (twice the 256 MB MALL by default), all sequences launched back to back
    through forward_into, captured once in a HIP graph and replayed.  Also
    the same launches eager (the Python API path of every call).  Returns
    µs per sequence and per GEMV and the effective weight bandwidth."""
    from .operators import int4gemv as op4
    from .operators import qgemv as op8
    mod, nbytes_of = ((op4, op4.int4_bytes) if op == "int4gemv"
                      else (op8, op8.q8_bytes))
    seq_bytes = sum(nbytes_of(N, K) for N, K in STRESS_SHAPES)
    nseq = max(2, -(-pool_bytes // seq_bytes))
    ext, variant = build(op), VARIANT[op]
    seqs = [[mod.device_random_set(N, K, 7919 * i + j)
             for j, (N, K) in enumerate(STRESS_SHAPES)] for i in range(nseq)]

    def all_sequences():
        for seq in seqs:
            for W, sc, x, out in seq:
                ext.forward_into(variant, W, sc, x, out)

    all_sequences()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=side):
        all_sequences()
    torch.cuda.synchronize()
    res = {"op": op, "variant": variant, "shapes": [list(s) for s in STRESS_SHAPES],
           "sequences_in_pool": nseq, "pool_bytes": nseq * seq_bytes,
           "bytes_per_sequence": seq_bytes,
           "note": "one replay runs every sequence of the pool once; each sequence "
                   "is six dependent-free launches on one stream"}
    for mode, fn in (("graph", g.replay), ("eager", all_sequences)):
        us = time_steps(fn, replays, warmup) / nseq
        res[mode] = {"us_per_sequence": round(us, 2),
                     "us_per_gemv": round(us / len(STRESS_SHAPES), 3),
                     "GBps": round(seq_bytes / us / 1e3, 1),
                     "frac_peak": round(seq_bytes / us / 1e3 / 8000.0, 4)}
    return res


def run(op: str = "int4gemv", layers: int | None = None, steps: int = 20,
        warmup: int = 3, modes=MODES, model: str = "7b") -> dict:
    cfg = MODELS[model]
    layers = cfg["layers"] if layers is None else layers
    m = DecodeModel(op, layers, hidden=cfg["hidden"], inter=cfg["inter"],
                    kv=cfg["kv"])
    graph = m.capture() if "graph" in modes else None
    res = {"op": op, "variant": m.variant, "model": model, "layers": layers,
           "hidden": m.hidden, "inter": m.inter, "kv": m.kv,
           "bytes_per_step": m.bytes_per_step,
           "launches_per_layer": {"sequential": 7, "grouped": 4, "graph": 4},
           "note": "sequential and grouped include the Python API path of "
                   "every call (forward_into and forward_grouped through "
                   "the checked-once fast path); graph replays the grouped "
                   "step's launches from one HIP graph"}
    fns = {"sequential": m.step_sequential, "grouped": m.step_grouped,
           "graph": graph.replay if graph is not None else None}
    for mode in modes:
        fn = fns[mode]
        us = time_steps(fn, steps, warmup)
        res[mode] = {"us_per_step": round(us, 2),
                     "us_per_layer": round(us / layers, 3),
                     "GBps": round(m.bytes_per_step / us / 1e3, 1),
                     "frac_peak": round(m.bytes_per_step / us / 1e3 / 8000.0, 4)}
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--op", choices=tuple(VARIANT), default="int4gemv")
    ap.add_argument("--model", choices=tuple(MODELS), default="7b")
    ap.add_argument("--layers", type=int, default=None,
                    help="layers (default: the model's, 32 for 7b, 80 for 70b)")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--modes", default=",".join(MODES),
                    help="comma-separated subset of " + ",".join(MODES))
    ap.add_argument("--stress", action="store_true",
                    help="time the decode stress sequence (11008x4096, 4096x11008, "
                         "4 x 4096x4096) over an HBM-cold pool instead of a model")
    a = ap.parse_args(argv)
    from . import _capi
    print(f"library: {_capi.version()}", flush=True)   # the build that ran
    if a.stress:
        if not torch.cuda.is_available():
            print("decode: no GPU visible", file=sys.stderr)
            return 1
        print(json.dumps(stress(a.op, a.steps, a.warmup)), flush=True)
        return 0
    modes = tuple(m for m in a.modes.split(",") if m)
    if not modes or any(m not in MODES for m in modes):
        print(f"decode: --modes must name some of {MODES}", file=sys.stderr)
        return 2
    if a.layers is not None and a.layers < 1:
        print("decode: --layers must be >= 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("decode: no GPU visible", file=sys.stderr)
        return 1
    print(json.dumps(run(a.op, a.layers, a.steps, a.warmup, modes, a.model)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
