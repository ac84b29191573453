"""The committed golden vectors (tests/golden/*.npz) are reproduced bit for
bit by the generator script (which runs the pinned oracle), and the product
quantizers reproduce the fixtures' packed weights and scales."""
from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import torch

from cudalab_amd.int4gemv_quantize import quantize_w as q4
from cudalab_amd.qgemv_quantize import quantize_w as q8
from oracle import oracle as orc

GOLDEN = Path(__file__).parent / "golden"


def _generator():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_fixtures_regenerate_bit_for_bit():
    fresh = _generator().make()
    for name, arrays in fresh.items():
        saved = np.load(GOLDEN / name)
        assert set(saved.files) == set(arrays), name
        for k, v in arrays.items():
            assert np.array_equal(saved[k], v, equal_nan=True), (name, k)


def test_product_quantizers_reproduce_fixtures():
    d = np.load(GOLDEN / "int4gemv_golden.npz")
    for i in range(int(d["n_cases"])):
        W = torch.from_numpy(d[f"w16_{i}"].view(np.float16))
        wp, s = q4(W)
        assert np.array_equal(wp.numpy(), d[f"wp_{i}"]), i
        assert np.array_equal(s.numpy().view(np.uint16), d[f"scale_{i}"]), i
    d = np.load(GOLDEN / "qgemv_golden.npz")
    for i in range(int(d["n_cases"])):
        W = torch.from_numpy(d[f"w16_{i}"].view(np.float16))
        wq, s = q8(W)
        assert np.array_equal(wq.numpy(), d[f"wq_{i}"]), i
        assert np.array_equal(s.numpy(), d[f"scale_{i}"]), i


def test_fixture_references_pass_their_own_bound():
    d = np.load(GOLDEN / "int4gemv_golden.npz")
    for i in range(int(d["n_cases"])):
        y = d[f"ref16_{i}"].view(np.float16)
        K = d[f"x_{i}"].size
        assert orc.arith_ratio(y, d[f"exact_{i}"], d[f"S_{i}"], K).max() <= 1.0
    d = np.load(GOLDEN / "qgemv_golden.npz")
    for i in range(int(d["n_cases"])):
        y = d[f"ref16_{i}"].view(np.float16)
        K = d[f"x_{i}"].size
        assert orc.arith_ratio(y, d[f"exact_{i}"], d[f"S_{i}"], K).max() <= 1.0
