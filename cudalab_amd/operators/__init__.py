"""Operator registry: `get(name)` returns the adapter singleton.

Drop-in for `cudalab/operators/__init__.py:17-29`, restricted to the
operators of the GEMV path ("int4gemv", "qgemv" and the FP16/FP32 "gemv")."""
from __future__ import annotations

from .gemv import gemv as _gemv
from .int4gemv import int4gemv as _int4gemv
from .qgemv import qgemv as _qgemv

_REGISTRY = {op.name: op for op in (_int4gemv, _qgemv, _gemv)}


def get(name: str):
    try:
        return _REGISTRY[name]
    except KeyError:
        raise KeyError(f"unknown operator {name!r}; available: "
                       f"{sorted(_REGISTRY)}") from None


def names() -> list[str]:
    return sorted(_REGISTRY)
