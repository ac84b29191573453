"""FP16/FP32 GEMV negative suite (per variant).

Drop-in for `cudalab/gemv_negative.py:67-351`: illegal inputs are rejected
before any launch with an explicit message; legal inputs (offset views
included) are never rejected; inputs that miss the vector contract (16-byte
aligned W and x, K a multiple of the elements per 16 bytes) run the scalar
kernel and are bit-identical to `gemv_baseline`.  After every case a
control forward checks that the device context is healthy.

Cases (24): W 8 (1d / 3d / N_zero / K_zero / bfloat16 / int32 / cpu /
transpose_view), unknown_variant, x 5 (len / 2d / dtype / cpu / noncontig),
out 4 (len / dtype / noncontig / cpu), controls 3 (forward_into, W offset
view, x offset view), fallback 3 (W +4 B, x +2 B, K = 13).  For the
quarantined `gemv_splitk4` (registered for callers that name it; it runs
the scalar kernel here) every fallback case holds bit-identically too.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from .evaluator.gpu import now_iso
from .evaluator.negative import run_case, summarize_cases
from .operators.gemv import make_w, make_x

SUITE_VERSION = "negative-gemv"
V = "gemv_baseline"


def _post_check_ok(ext, variant: str = V) -> bool:
    try:
        torch.cuda.synchronize()
        W = make_w(2, 16, torch.float16, seed=11)
        x = make_x(16, torch.float16, seed=12)
        y = ext.forward(variant, W, x)
        torch.cuda.synchronize()
        return bool(torch.isfinite(y.float()).all())
    except Exception:  # noqa: BLE001
        return False


def build_cases(ext, variant: str = V) -> list[dict]:
    dev = "cuda"
    cases: list[dict] = []

    def add(cid, description, call, expected="reject",
            expect_msg_contains=None):
        cases.append(dict(id=cid, variant=variant, description=description,
                          call=call, expected=expected,
                          expect_msg_contains=expect_msg_contains))

    N, K = 8, 64
    W = make_w(N, K, torch.float16, device=dev, seed=0)
    x = make_x(K, torch.float16, device=dev, seed=1)
    fwd = lambda Wa, xa: ext.forward(variant, Wa, xa)  # noqa: E731

    # ---- W
    add("W_1d", "W is 1-D (N*K,)",
        lambda: fwd(torch.randn(N * K, dtype=torch.float16, device=dev), x),
        expect_msg_contains="必须是 2 维")
    add("W_3d", "W is 3-D (2, 4, 8)",
        lambda: fwd(torch.randn(2, 4, 8, dtype=torch.float16, device=dev), x),
        expect_msg_contains="必须是 2 维")
    add("W_N_zero", "N = 0",
        lambda: fwd(torch.empty(0, K, dtype=torch.float16, device=dev), x),
        expect_msg_contains="N 必须 > 0")
    add("W_K_zero", "K = 0",
        lambda: fwd(torch.empty(N, 0, dtype=torch.float16, device=dev), x),
        expect_msg_contains="K 必须 > 0")
    add("W_bfloat16", "W is bfloat16 (fp16 / fp32 only)",
        lambda: fwd(make_w(N, K, torch.bfloat16, device=dev, seed=0), x),
        expect_msg_contains="float16 / float32")
    add("W_int32", "W is int32",
        lambda: fwd(torch.randint(-3, 3, (N, K), dtype=torch.int32, device=dev), x),
        expect_msg_contains="float16 / float32")
    add("W_cpu", "W on the CPU",
        lambda: fwd(make_w(N, K, torch.float16, device="cpu", seed=0), x),
        expect_msg_contains="CUDA 张量")
    add("W_transpose_view", "W is a (K, N).t() view (not contiguous)",
        lambda: fwd(make_w(K, N, torch.float16, device=dev, seed=1).t(), x),
        expect_msg_contains="连续内存")
    add("unknown_variant", "unknown variant name",
        lambda: ext.forward("no_such_gemv_variant", W, x),
        expect_msg_contains="未知 gemv 变体")

    # ---- x
    add("x_len_mismatch", "x length K-1",
        lambda: fwd(W, make_x(K - 1, torch.float16, device=dev, seed=2)),
        expect_msg_contains="长度必须等于 K")
    add("x_2d", "x is 2-D (1, K)",
        lambda: fwd(W, x.view(1, K)),
        expect_msg_contains="必须是 1 维")
    add("x_dtype_mismatch", "x float32 with W float16",
        lambda: fwd(W, x.float()),
        expect_msg_contains="dtype 必须与 W 一致")
    add("x_cpu", "x on the CPU",
        lambda: fwd(W, x.cpu()),
        expect_msg_contains="CUDA 张量")
    add("x_noncontig", "x is a stride-2 view",
        lambda: fwd(W, make_x(2 * K, torch.float16, device=dev, seed=3)[::2]),
        expect_msg_contains="连续内存")

    # ---- out
    add("out_len_mismatch", "out length N+1",
        lambda: ext.forward_into(variant, W, x,
                                 torch.empty(N + 1, dtype=torch.float16, device=dev)),
        expect_msg_contains="长度必须等于 N")
    add("out_dtype_mismatch", "out float32 with W float16",
        lambda: ext.forward_into(variant, W, x,
                                 torch.empty(N, dtype=torch.float32, device=dev)),
        expect_msg_contains="dtype 必须与 W 一致")
    add("out_noncontig", "out is a stride-2 view",
        lambda: ext.forward_into(variant, W, x,
                                 torch.empty(2 * N, dtype=torch.float16, device=dev)[::2]),
        expect_msg_contains="连续内存")
    add("out_cpu", "out on the CPU",
        lambda: ext.forward_into(variant, W, x,
                                 torch.empty(N, dtype=torch.float16)),
        expect_msg_contains="CUDA 张量")

    # ---- controls: legal inputs are never rejected
    out_ok = torch.empty(N, dtype=torch.float16, device=dev)
    add("valid_forward_into_control", "control: legal forward_into must pass",
        lambda: ext.forward_into(variant, W, x, out_ok), expected="pass")
    big_w = torch.randn(N * K + 2, dtype=torch.float16, device=dev)
    Wo = big_w[2:2 + N * K].view(N, K)            # base + 4 B
    xo = make_x(K, torch.float16, device=dev, seed=5)

    def _offset_control():
        ext.forward_into(variant, Wo, xo, out_ok)
        assert torch.isfinite(out_ok.float()).all(), "offset-view output not finite"

    add("valid_offset_view_control",
        "control: W a contiguous view 2 elements (4 B) past the base: legal, "
        "must pass", _offset_control, expected="pass")
    big_x = torch.randn(K + 1, dtype=torch.float16, device=dev)
    add("valid_offset_view_x",
        "control: x a contiguous slice 1 element (2 B) past the base: legal, "
        "must pass", lambda: fwd(W, big_x[1:1 + K]), expected="pass")

    # ---- fallback: bit-identical to gemv_baseline
    def _fallback(cid, Wm, xm, n):
        out_f = torch.empty(n, dtype=Wm.dtype, device=dev)
        ext.forward_into(variant, Wm, xm, out_f)
        torch.cuda.synchronize()
        base = ext.forward("gemv_baseline", Wm, xm)
        torch.cuda.synchronize()
        assert torch.equal(out_f, base), (
            f"{cid}: output differs from gemv_baseline (the scalar kernel is "
            "the single source of every fallback)")

    big_w8 = torch.randn(N * K + 2, dtype=torch.float16, device=dev)
    Wm = big_w8[2:2 + N * K].view(N, K)
    Wa = make_w(N, K, torch.float16, device=dev, seed=7)
    xa = make_x(K, torch.float16, device=dev, seed=6)
    big_x8 = torch.randn(K + 1, dtype=torch.float16, device=dev)
    xm = big_x8[1:1 + K]
    add("fallback_W_misaligned",
        "fallback: W 4 B past a 16-byte boundary, x aligned, K % 8 == 0: "
        "contract unmet -> scalar kernel, bit-identical to gemv_baseline",
        lambda: _fallback("fallback_W_misaligned", Wm, xa, N), expected="pass")
    add("fallback_x_misaligned",
        "fallback: x 2 B past a 16-byte boundary, W aligned: contract unmet "
        "-> scalar kernel, bit-identical to gemv_baseline",
        lambda: _fallback("fallback_x_misaligned", Wa, xm, N), expected="pass")
    Wk = make_w(16, 13, torch.float16, device=dev, seed=8)
    xk = make_x(13, torch.float16, device=dev, seed=9)
    add("fallback_K_not_mult8",
        "fallback: K = 13 (not a multiple of 8): contract unmet -> scalar "
        "kernel, bit-identical to gemv_baseline",
        lambda: _fallback("fallback_K_not_mult8", Wk, xk, 16), expected="pass")
    return cases


def run_negative_suite(ext, out_path: Path | None = None,
                       variant: str = V) -> dict:
    cases = build_cases(ext, variant)
    results = []
    for c in cases:
        r = run_case(c["variant"], c["description"], c["call"], c["expected"],
                     c["expect_msg_contains"],
                     lambda v=c["variant"]: _post_check_ok(ext, v))
        r["id"] = c["id"]
        results.append(r)
    doc = {
        "suite": SUITE_VERSION,
        "negative_suite_scope": "per-variant",
        "generated": now_iso(),
        "note": ("illegal inputs are rejected before launch; inputs missing "
                 "the vector contract (16-byte aligned W and x, K a multiple "
                 "of the elements per 16 bytes) run the scalar kernel and are "
                 "bit-identical to gemv_baseline; legal inputs (offset views "
                 "included) are never rejected"),
        "summary": summarize_cases(results),
        "cases": results,
    }
    if out_path is not None:
        out_path = Path(out_path)
        out_path.parent.mkdir(parents=True, exist_ok=True)
        out_path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
    return doc
