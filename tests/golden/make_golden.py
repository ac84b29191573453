"""Writes the committed golden vectors of the GEMV path (tests/golden/*.npz).

Inputs come from numpy's seeded generator; quantization, exact row sums and
bound denominators come from the CPU oracle (oracle/), which is pinned by
tests/test_oracle_pins.py.  The reference holds no golden output vectors
(its correctness records store metrics only), so these fixtures freeze the
pinned oracle's answers: re-running this script must reproduce them bit for
bit (tests/test_golden.py checks that).

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as orc  # noqa: E402

HERE = Path(__file__).resolve().parent

INT4_SHAPES = [(1, 128), (3, 128), (8, 128), (16, 256), (1, 4096), (33, 384)]
INT8_SHAPES = [(1, 1), (16, 13), (8, 7), (1, 4096), (64, 48), (4096, 1)]
MODES = ("normal", "zeros", "tiny", "large", "mixed_sign")


def _w(rng, N, K, mode):
    if mode == "normal":
        w = rng.standard_normal((N, K)) * 0.02
    elif mode == "zeros":
        w = np.zeros((N, K))
    elif mode == "tiny":
        w = rng.standard_normal((N, K)) * 1e-4
    elif mode == "large":
        w = rng.standard_normal((N, K)) * 10
    else:
        w = np.abs(rng.standard_normal((N, K)))
        w *= np.where((np.arange(N)[:, None] + np.arange(K)[None, :]) % 2, -1, 1)
    return w.astype(np.float16)


def _x(rng, K, mode):
    if mode == "zeros":
        return np.zeros(K, np.float16)
    s = {"normal": 1.0, "tiny": 1e-4, "large": 10.0, "mixed_sign": 1.0}[mode]
    x = rng.standard_normal(K) * s
    if mode == "mixed_sign":
        x = np.abs(x) * np.where(rng.integers(0, 2, K) == 0, 1, -1)
    return x.astype(np.float16)


def make() -> dict[str, dict]:
    out = {}
    d4 = {}
    i = 0
    for (N, K) in INT4_SHAPES:
        for mi, mode in enumerate(MODES):
            rng = np.random.default_rng(1000 * N + K + mi)
            W = _w(rng, N, K, mode)
            x = _x(rng, K, mode)
            wp, s = orc.quantize_w4(W)
            ex, S = orc.exact_w4(wp, s, x)
            _, y16 = orc.ref_f32_w4(wp, s, x)
            d4.update({f"w16_{i}": W.view(np.uint16), f"wp_{i}": wp,
                       f"scale_{i}": s.view(np.uint16),
                       f"x_{i}": x.view(np.uint16), f"exact_{i}": ex,
                       f"S_{i}": S, f"ref16_{i}": y16.view(np.uint16)})
            i += 1
    d4["n_cases"] = np.array(i)
    out["int4gemv_golden.npz"] = d4
    d8 = {}
    i = 0
    for (N, K) in INT8_SHAPES:
        for mi, mode in enumerate(MODES):
            rng = np.random.default_rng(2000 * N + K + mi)
            W = _w(rng, N, K, mode)
            x = _x(rng, K, mode)
            wq, s = orc.quantize_w8(W)
            ex, S = orc.exact_w8(wq, s, x)
            _, y16 = orc.ref_f32_w8(wq, s, x)
            d8.update({f"w16_{i}": W.view(np.uint16), f"wq_{i}": wq,
                       f"scale_{i}": s, f"x_{i}": x.view(np.uint16),
                       f"exact_{i}": ex, f"S_{i}": S,
                       f"ref16_{i}": y16.view(np.uint16)})
            i += 1
    d8["n_cases"] = np.array(i)
    out["qgemv_golden.npz"] = d8
    return out


if __name__ == "__main__":
    for name, arrays in make().items():
        np.savez_compressed(HERE / name, **arrays)
        print(f"wrote {HERE / name} ({arrays['n_cases']} cases)")
