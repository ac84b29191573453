"""Negative-case runner, shared by the INT4, INT8 and FP16/FP32 suites.

The contract of the reference's runner (cudalab/evaluator/negative.py:23-84),
whose record keys the suites' JSON keeps: a case is a callable that is
expected to raise before anything is launched ("reject", optionally with a
substring its message must contain), to complete ("pass"), or is called but
not judged ("skip").  After every judged case a control callback launches a
known good call and checks its result, so a case that left the device
unusable fails even if it raised as expected.
"""
from __future__ import annotations

from collections import Counter
from dataclasses import dataclass
from typing import Callable, Optional

import torch

_MSG_CHARS = 300


@dataclass(frozen=True)
class _Attempt:
    """What calling a case did: whether it raised, and what."""
    raised: bool
    exc_type: Optional[str] = None
    message: Optional[str] = None

    @property
    def status(self) -> str:
        return "rejected" if self.raised else "passed_without_exception"


def _attempt(call: Callable[[], None]) -> _Attempt:
    try:
        call()
    except Exception as e:  # noqa: BLE001 -- any exception counts as a rejection
        first = (str(e).splitlines() or [""])[0]
        return _Attempt(True, type(e).__name__, first[:_MSG_CHARS])
    return _Attempt(False)


def _passes(expected: str, a: _Attempt, msg_match: Optional[bool],
            healthy: bool) -> bool:
    """The pass rule: the device is healthy afterwards, and a "reject" case
    raised (with the expected message, when one is given) while a "pass"
    case did not raise."""
    if not healthy:
        return False
    if expected == "reject":
        return a.raised and msg_match is not False
    return not a.raised


def run_case(variant: str, description: str, call: Callable[[], None],
             expected: str, expect_msg_contains: Optional[str],
             control_ok: Callable[[], bool]) -> dict:
    """Run one case (expected "reject" | "pass" | "skip") and return its
    record."""
    if torch.cuda.is_available():
        torch.cuda.synchronize()      # earlier work must not leak into the case
    a = _attempt(call)
    match = (expect_msg_contains in a.message
             if expect_msg_contains and a.message else None)
    rec = {"variant": variant, "description": description,
           "expected": expected, "status": a.status,
           "exception_type": a.exc_type, "message": a.message,
           "expect_msg_contains": expect_msg_contains, "msg_match": match,
           "post_check_ok": None}
    if expected == "skip":
        rec["status"] = "skipped"
        return rec
    healthy = bool(control_ok())
    rec["post_check_ok"] = healthy
    rec["pass"] = _passes(expected, a, match, healthy)
    return rec


def summarize_cases(results: list[dict]) -> dict:
    """Counts per expectation and the suite verdict (skipped cases do not
    count against it)."""
    by = Counter((r["expected"], bool(r.get("pass"))) for r in results)
    expected = Counter(r["expected"] for r in results)
    return {
        "n_total": len(results),
        "n_reject_expected": expected["reject"],
        "n_reject_ok": by[("reject", True)],
        "n_pass_expected": expected["pass"],
        "n_pass_ok": by[("pass", True)],
        "n_skipped": expected["skip"],
        "n_passed": sum(n for (_, ok), n in by.items() if ok),
        "all_pass": all(r.get("pass") for r in results if r["expected"] != "skip"),
    }
