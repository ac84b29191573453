"""Decode-step driver: the seven weight projections of every layer of a
Llama-7B-shaped model, back to back on one GPU, through the INT4 (or INT8)
GEMV path.  No counterpart in the reference (it excludes model
integration: README.md:34-35); this restates the "back-to-back Llama-7B
decode projections" workload of the benchmark configuration.

Per layer, hidden H = 4096 and intermediate I = 11008:
  q, k, v   H -> H   from the layer input       (independent: one group)
  o         H -> H   from v                     (a single-token context makes
                                                 attention the identity on v)
  gate, up  H -> I   from o                     (independent: one group)
  down      I -> H   from up                    (feeds the next layer)
Norms, attention over a longer context, the residual adds and the SwiGLU
product are outside the GEMV path and are not modelled; the data
dependencies between projections follow the layer's order.

Weights are random-init: W ~ N(0, 1/K) in fp16 (so activations stay O(1)
through all layers), quantized with the path's own quantizers on the
device.  Three ways to run one decode step over all layers:
  sequential  one launch per projection (7 per layer)
  grouped     q/k/v and gate/up as grouped launches (4 per layer)
  graph       the grouped step captured once in a HIP graph and replayed
All three produce bit-identical outputs.

Usage: python -m cudalab_amd.decode [--layers 32] [--op int4gemv]
       [--steps 20] [--warmup 3] [--modes sequential,grouped,graph]
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
VARIANT = {"int4gemv": "int4gemv_cdna4", "qgemv": "qgemv_cdna4"}
PROJ = (("q", HIDDEN, HIDDEN), ("k", HIDDEN, HIDDEN), ("v", HIDDEN, HIDDEN),
        ("o", HIDDEN, HIDDEN), ("gate", INTER, HIDDEN), ("up", INTER, HIDDEN),
        ("down", HIDDEN, INTER))


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
                 hidden: int = HIDDEN, inter: int = INTER):
        self.op = op
        self.ext = build(op)
        self.variant = VARIANT[op]
        self.hidden, self.inter = hidden, inter
        self.proj = tuple((n, (hidden if a == HIDDEN else inter),
                           (hidden if b == HIDDEN else inter))
                          for (n, a, b) in PROJ)
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

    def step_sequential(self) -> torch.Tensor:
        x = self.x0
        for L in self.layers:
            for n in ("q", "k", "v"):
                self._one(L, n, x)
            self._one(L, "o", L.out["v"])
            for n in ("gate", "up"):
                self._one(L, n, L.out["o"])
            self._one(L, "down", L.out["up"])
            x = L.out["down"]
        return x

    def step_grouped(self) -> torch.Tensor:
        x = self.x0
        for L in self.layers:
            self._group(L, ("q", "k", "v"), x)
            self._one(L, "o", L.out["v"])
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


def run(op: str = "int4gemv", layers: int = LAYERS, steps: int = 20,
        warmup: int = 3, modes=MODES) -> dict:
    m = DecodeModel(op, layers)
    graph = m.capture() if "graph" in modes else None
    res = {"op": op, "variant": m.variant, "layers": layers,
           "bytes_per_step": m.bytes_per_step,
           "launches_per_layer": {"sequential": 7, "grouped": 4, "graph": 4},
           "note": "sequential and grouped include the Python API path of "
                   "every call (validation, ctypes); graph replays the "
                   "grouped step's launches from one HIP graph"}
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
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--modes", default=",".join(MODES),
                    help="comma-separated subset of " + ",".join(MODES))
    a = ap.parse_args(argv)
    modes = tuple(m for m in a.modes.split(",") if m)
    if not modes or any(m not in MODES for m in modes):
        print(f"decode: --modes must name some of {MODES}", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("decode: no GPU visible", file=sys.stderr)
        return 1
    print(json.dumps(run(a.op, a.layers, a.steps, a.warmup, modes)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
