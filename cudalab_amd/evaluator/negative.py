"""Negative-case runner (operator-agnostic).

Drop-in for `cudalab/evaluator/negative.py:23-84`: a case is a callable
that must either raise before any launch (expected "reject", optionally with
a message substring) or succeed (expected "pass"); after every non-skipped
case a control callback checks that the device context is still healthy.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch


def run_case(variant: str, description: str, call: Callable[[], None],
             expected: str, expect_msg_contains: Optional[str],
             control_ok: Callable[[], bool]) -> dict:
    """Run one case; expected is "reject" | "pass" | "skip"."""
    torch.cuda.synchronize()
    status = "rejected"
    exc_type = None
    message = None
    try:
        call()
        status = "passed_without_exception"
    except Exception as e:  # noqa: BLE001 -- any exception is a rejection
        exc_type = type(e).__name__
        message = (str(e).splitlines() or [""])[0][:300]
    rec = {
        "variant": variant,
        "description": description,
        "expected": expected,
        "status": status,
        "exception_type": exc_type,
        "message": message,
        "expect_msg_contains": expect_msg_contains,
        "msg_match": (expect_msg_contains in message)
        if (expect_msg_contains and message) else None,
        "post_check_ok": None,
    }
    if expected == "skip":
        rec["status"] = "skipped"
        return rec
    rec["post_check_ok"] = bool(control_ok())
    if expected == "reject":
        rec["pass"] = (status == "rejected" and rec["post_check_ok"]
                       and rec["msg_match"] is not False)
    else:
        rec["pass"] = (status == "passed_without_exception"
                       and rec["post_check_ok"])
    return rec


def summarize_cases(results: list[dict]) -> dict:
    rej = [r for r in results if r["expected"] == "reject"]
    ok = [r for r in results if r["expected"] == "pass"]
    skipped = [r for r in results if r["expected"] == "skip"]
    return {
        "n_total": len(results),
        "n_reject_expected": len(rej),
        "n_reject_ok": sum(1 for r in rej if r.get("pass")),
        "n_pass_expected": len(ok),
        "n_pass_ok": sum(1 for r in ok if r.get("pass")),
        "n_skipped": len(skipped),
        "n_passed": sum(1 for r in results if r.get("pass")),
        "all_pass": all(r.get("pass") for r in results
                        if r["expected"] != "skip"),
    }
