"""Crafted fp16 weight matrices for the quantizer tests (CPU and GPU): exact
round-half-even ties of w / s, values one fp16 step either side of a tie,
fp16 subnormals, zero and signed-zero groups, the amax at every position
and sign, the fp16 extremes, and plain seeded random rows.  Each builder
returns a float16 numpy array (N, K) with K % 128 == 0."""
from __future__ import annotations

import numpy as np

G = 128


def _rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def ties(qmax: int, n_groups: int, seed: int, k: int = G) -> np.ndarray:
    """Groups whose amax is qmax * 2^e (so s = amax / qmax = 2^e exactly)
    and whose other entries are (j + 1/2) * 2^e: every w / s is an exact
    tie, which round-half-even sends to the even neighbour."""
    r = _rng(seed)
    rows = []
    for i in range(n_groups):
        e = int(r.integers(-14, 8)) if qmax == 7 else int(r.integers(-14, 2))
        j = r.integers(-qmax, qmax, size=k).astype(np.float64) + 0.5
        v = j * 2.0 ** e
        v[int(r.integers(0, k))] = qmax * 2.0 ** e * (1 if i % 2 else -1)
        rows.append(v)
    return np.asarray(rows, dtype=np.float16)


def near_ties(qmax: int, n_groups: int, seed: int, k: int = G) -> np.ndarray:
    """As `ties`, with each tie moved one fp16 step up or down."""
    t = ties(qmax, n_groups, seed, k)
    bits = t.view(np.uint16).copy()
    r = _rng(seed + 1)
    step = r.choice(np.array([-1, 1], dtype=np.int32), size=bits.shape)
    amax = np.abs(t.astype(np.float32)).max(axis=1, keepdims=True)
    keep = np.abs(t.astype(np.float32)) == amax        # leave the amax alone
    moved = (bits.astype(np.int32) + np.where(keep, 0, step)).astype(np.uint16)
    out = moved.view(np.float16)
    # a step past the amax's magnitude would change s; clip those back
    over = np.abs(out.astype(np.float32)) > amax
    out[over] = t[over]
    return out


def subnormals(n: int, k: int, seed: int) -> np.ndarray:
    """Values that are fp16 subnormals (multiples of 2^-24 below 2^-14)."""
    r = _rng(seed)
    m = r.integers(-1023, 1024, size=(n, k)).astype(np.float64)
    return (m * 2.0 ** -24).astype(np.float16)


def zero_groups(n: int, k: int, seed: int) -> np.ndarray:
    """Random rows in which about a third of the groups are +0 and a third
    are -0 (a signed zero group is still a zero group)."""
    r = _rng(seed)
    W = r.standard_normal((n, k)).astype(np.float16)
    g = W.reshape(n, k // G, G)
    pick = r.integers(0, 3, size=(n, k // G))
    g[pick == 1] = np.float16(0.0)
    g[pick == 2] = np.float16(-0.0)
    return g.reshape(n, k)


def amax_positions(k: int = G) -> np.ndarray:
    """Row r (0 <= r < 256) has its largest magnitude, 3.0 with the sign
    (-1)^r, at column r // 2: each position of the first group holds the
    amax once with each sign; the other entries are 0.25 and -0.125."""
    n = 2 * G
    W = np.full((n, k), 0.25, dtype=np.float16)
    W[:, 1::2] = np.float16(-0.125)
    for r_ in range(n):
        pos = r_ // 2
        W[r_, pos] = np.float16(3.0 if r_ % 2 == 0 else -3.0)
    return W


def extremes(k: int = G) -> np.ndarray:
    """fp16 extremes: +-65504, the smallest subnormal, the smallest normal,
    and one-nonzero groups."""
    rows = []
    a = np.zeros(k, dtype=np.float16); a[0] = 65504; a[1] = -65504; a[2] = 1; rows.append(a)
    b = np.zeros(k, dtype=np.float16); b[5] = np.float16(2.0 ** -24); rows.append(b)
    c = np.zeros(k, dtype=np.float16); c[7] = -np.float16(2.0 ** -24); c[8] = np.float16(2.0 ** -25 * 1.0); rows.append(c)
    d = np.full(k, np.float16(2.0 ** -14)); d[::3] = -np.float16(2.0 ** -14); rows.append(d)
    e = np.linspace(-65504, 65504, k).astype(np.float16); rows.append(e)
    f = np.zeros(k, dtype=np.float16); f[-1] = np.float16(1e-3); rows.append(f)
    return np.stack(rows)


def random_rows(n: int, k: int, seed: int, std: float = 1.0) -> np.ndarray:
    return (_rng(seed).standard_normal((n, k)) * std).astype(np.float16)


def all_cases(qmax: int) -> dict[str, np.ndarray]:
    """The crafted set for one quantizer (qmax = 7 for INT4, 127 for INT8)."""
    return {
        "ties": ties(qmax, 96, seed=11),
        "near_ties": near_ties(qmax, 96, seed=12),
        "subnormals": subnormals(16, 4 * G, seed=13),
        "zero_groups": zero_groups(24, 8 * G, seed=14),
        "amax_positions": amax_positions(),
        "extremes": extremes(),
        "random": random_rows(64, 8 * G, seed=15),
        "random_small": random_rows(32, 4 * G, seed=16, std=0.02),
    }
