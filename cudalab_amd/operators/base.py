"""Operator adapter protocol: the boundary between an operator and the
evaluation tools.  Drop-in for `cudalab/operators/base.py:40-118`."""
from __future__ import annotations

from pathlib import Path

import torch

from ..evaluator.bench import BenchPool  # noqa: F401  (re-export)


class Operator:
    """Subclasses declare: name, dtypes, bench_shapes, primary_target,
    kernel_regex (also as ncu_kernel_regex), profiles_dir, bench_dir,
    experiments_dir."""
    name: str
    dtypes: tuple
    bench_shapes: list
    primary_target: tuple
    kernel_regex: str
    ncu_kernel_regex: str
    profiles_dir: Path
    bench_dir: Path
    experiments_dir: Path

    def build(self):
        raise NotImplementedError

    def variants(self, ext) -> list[str]:
        """Dispatchable variants (quarantined ones excluded)."""
        return sorted(ext.variants())

    def unsafe_variants(self, ext) -> list[str]:
        """Quarantined variants: registered, hidden from variants()."""
        fn = getattr(ext, "quarantined_variants", None)
        return sorted(fn()) if fn is not None else []

    def make_bench_pool(self, M: int, H: int, dtype: torch.dtype, mode: str,
                        seed: int, pool_size: int) -> BenchPool:
        raise NotImplementedError

    def algorithmic_bytes(self, M: int, H: int, element_size: int) -> int:
        raise NotImplementedError

    def profile_driver_source(self, variant: str, M: int, H: int) -> str:
        raise NotImplementedError

    def ncu_driver_source(self, variant: str, M: int, H: int) -> str:
        """Name kept from the reference protocol; the driver is
        profiler-agnostic (used with rocprofv3 on MI355X)."""
        return self.profile_driver_source(variant, M, H)

    def pytorch_ref_latency(self, M: int, H: int, dtype: torch.dtype,
                            iters: int = 200, batch: int = 32) -> dict:
        raise NotImplementedError

    def experiment_prefix(self) -> str:
        raise NotImplementedError

    def run_correctness(self, ext, variant: str,
                        out_dir: Path | None = None) -> dict:
        raise NotImplementedError

    def run_negative(self, ext, variant: str | None = None,
                     out_dir: Path | None = None) -> dict:
        raise NotImplementedError
