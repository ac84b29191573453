"""INT8 W8A16 GEMV negative suite (per variant).

Drop-in for `cudalab/qgemv_negative.py:62-330`: 29 cases (W_q 8, scale 5,
x 5, out 4, variant 1, control 3, fallback 3).  The vector contract is
16-byte aligned W_q and x with K % 16 == 0; inputs that miss it (including
K = 13) run the scalar kernel, bit-identical to `qgemv_baseline`.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from .evaluator.gpu import now_iso
from .evaluator.negative import run_case, summarize_cases
from .operators.qgemv import make_w_q, make_x_q

SUITE_VERSION = "negative-qgemv"
V = "qgemv_baseline"


def _post_check_ok(ext, variant: str = V) -> bool:
    try:
        torch.cuda.synchronize()
        W_q, scale, _ = make_w_q(2, 16, seed=0)
        x = make_x_q(16, seed=1)
        y = ext.forward(variant, W_q, scale, x)
        torch.cuda.synchronize()
        return bool(torch.isfinite(y.float()).all())
    except Exception:  # noqa: BLE001
        return False


def _rand_q(shape, seed: int, device: str = "cuda") -> torch.Tensor:
    """Random int8 in [-127, 127]."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g,
                         dtype=torch.int8).to(device)


def build_cases(ext, variant: str = V) -> list[dict]:
    dev = "cuda"
    cases: list[dict] = []

    def add(cid, description, call, expected="reject",
            expect_msg_contains=None):
        cases.append(dict(id=cid, variant=variant, description=description,
                          call=call, expected=expected,
                          expect_msg_contains=expect_msg_contains))

    N, K = 8, 64
    W_q, scale, _ = make_w_q(N, K, seed=0)
    x = make_x_q(K, seed=1)

    def fwd(Wa, sa, xa):
        return ext.forward(variant, Wa, sa, xa)

    # ---- W_q ----
    w_1d = _rand_q((N * K,), 2)
    add("W_q_1d", "W_q is 1-D", lambda: fwd(w_1d, scale, x),
        expect_msg_contains="必须是 2 维")
    w_3d = _rand_q((N, K), 3).view(2, N // 2, K)
    add("W_q_3d", "W_q is 3-D", lambda: fwd(w_3d, scale, x),
        expect_msg_contains="必须是 2 维")
    w_n0 = torch.empty(0, K, dtype=torch.int8, device=dev)
    add("W_q_N_zero", "N = 0", lambda: fwd(w_n0, scale[:0].contiguous(), x),
        expect_msg_contains="N 必须 > 0")
    w_k0 = torch.empty(N, 0, dtype=torch.int8, device=dev)
    add("W_q_K_zero", "K = 0", lambda: fwd(w_k0, scale, x),
        expect_msg_contains="K 必须 > 0")
    w_f16 = torch.randn(N, K, dtype=torch.float16, device=dev)
    add("W_q_dtype_fp16", "W_q is fp16 (must be int8)",
        lambda: fwd(w_f16, scale, x), expect_msg_contains="必须是 int8")
    w_i32 = torch.randint(-3, 3, (N, K), dtype=torch.int32, device=dev)
    add("W_q_dtype_int32", "W_q is int32 (must be int8)",
        lambda: fwd(w_i32, scale, x), expect_msg_contains="必须是 int8")
    w_cpu = _rand_q((N, K), 4, device="cpu")
    add("W_q_cpu", "W_q on the CPU",
        lambda: fwd(w_cpu, scale.cpu(), x.cpu()),
        expect_msg_contains="CUDA 张量")
    w_t = _rand_q((K, N), 5).t()
    add("W_q_noncontig", "W_q is a transposed (non-contiguous) view",
        lambda: fwd(w_t, scale, x), expect_msg_contains="连续内存")

    # ---- scale ----
    s_short = scale[:N - 1].contiguous()
    add("scale_len_mismatch", "scale has N - 1 elements",
        lambda: fwd(W_q, s_short, x),
        expect_msg_contains="scale 长度必须等于 N")
    s_2d = scale.view(N, 1)
    add("scale_2d", "scale is 2-D (N, 1)", lambda: fwd(W_q, s_2d, x),
        expect_msg_contains="必须是 1 维")
    s_f16 = scale.half()
    add("scale_dtype_fp16", "scale is fp16 (must be fp32)",
        lambda: fwd(W_q, s_f16, x), expect_msg_contains="必须是 float32")
    add("scale_cpu", "scale on the CPU", lambda: fwd(W_q, scale.cpu(), x),
        expect_msg_contains="CUDA 张量")
    s_big = torch.randn(2 * N, dtype=torch.float32, device=dev)
    s_nc = s_big[::2]
    add("scale_noncontig", "scale is a stride-2 slice",
        lambda: fwd(W_q, s_nc, x), expect_msg_contains="连续内存")

    # ---- x ----
    x_short = make_x_q(K - 1, seed=6)
    add("x_len_mismatch", "x has K - 1 elements",
        lambda: fwd(W_q, scale, x_short),
        expect_msg_contains="x 长度必须等于 K")
    x_2d = x.view(1, K)
    add("x_2d", "x is 2-D", lambda: fwd(W_q, scale, x_2d),
        expect_msg_contains="必须是 1 维")
    x_f32 = make_x_q(K, seed=7).float()
    add("x_dtype_fp32", "x is fp32 (must be fp16)",
        lambda: fwd(W_q, scale, x_f32), expect_msg_contains="必须是 float16")
    add("x_cpu", "x on the CPU", lambda: fwd(W_q, scale, x.cpu()),
        expect_msg_contains="CUDA 张量")
    x_big = torch.randn(2 * K, dtype=torch.float16, device=dev)
    x_nc = x_big[::2]
    add("x_noncontig", "x is a stride-2 slice",
        lambda: fwd(W_q, scale, x_nc), expect_msg_contains="连续内存")

    # ---- out ----
    add("out_wrong_shape", "out has N - 1 elements",
        lambda: ext.forward_into(variant, W_q, scale, x,
                                 torch.empty(N - 1, dtype=torch.float16,
                                             device=dev)),
        expect_msg_contains="out 长度必须等于 N")
    add("out_wrong_dtype", "out is fp32",
        lambda: ext.forward_into(variant, W_q, scale, x,
                                 torch.empty(N, dtype=torch.float32,
                                             device=dev)),
        expect_msg_contains="必须是 float16")
    o_big = torch.randn(2 * N, dtype=torch.float16, device=dev)
    o_nc = o_big[::2]
    add("out_noncontig", "out is a stride-2 slice",
        lambda: ext.forward_into(variant, W_q, scale, x, o_nc),
        expect_msg_contains="连续内存")
    add("out_cpu", "out on the CPU",
        lambda: ext.forward_into(variant, W_q, scale, x,
                                 torch.empty(N, dtype=torch.float16)),
        expect_msg_contains="CUDA 张量")

    # ---- variant ----
    add("unknown_variant", "unknown variant name",
        lambda: ext.forward("no_such_qgemv_variant", W_q, scale, x),
        expect_msg_contains="未知 qgemv 变体")

    # ---- controls ----
    out_ok = torch.empty(N, dtype=torch.float16, device=dev)
    add("valid_forward_into_control", "control: legal forward_into succeeds",
        lambda: ext.forward_into(variant, W_q, scale, x, out_ok),
        expected="pass")
    big_wq = _rand_q((N * K + 16,), 8)
    Wq_mis = big_wq[1:1 + N * K].view(N, K)            # base + 1 byte

    def _wq_offset_control():
        ext.forward_into(variant, Wq_mis, scale, x, out_ok)
        y = ext.forward(variant, W_q, scale, x)
        assert torch.isfinite(out_ok.float()).all(), "offset-view output not finite"
        assert torch.isfinite(y.float()).all(), "control output not finite"

    add("valid_offset_view_Wq_control",
        "control: W_q is a contiguous view 1 byte past a 16-byte boundary; "
        "legal, must succeed", _wq_offset_control, expected="pass")
    big_xv = torch.randn(K + 8, dtype=torch.float16, device=dev)
    xo_mis = big_xv[1:1 + K]                           # base + 2 bytes
    add("valid_offset_view_x_control",
        "control: x is a contiguous slice 2 bytes past a 16-byte boundary; "
        "legal, must succeed", lambda: fwd(W_q, scale, xo_mis),
        expected="pass")

    # ---- fallback: bit-identical to qgemv_baseline ----
    def _fallback_check(cid, Wm, sm, xm):
        out_f = torch.empty(Wm.size(0), dtype=torch.float16, device=dev)
        ext.forward_into(variant, Wm, sm, xm, out_f)
        torch.cuda.synchronize()
        y_base = ext.forward("qgemv_baseline", Wm, sm, xm)
        torch.cuda.synchronize()
        assert torch.equal(out_f, y_base), (
            f"{cid}: fallback output differs from qgemv_baseline (must be "
            "bit-identical: same scalar kernel)")

    xa = make_x_q(K, seed=9)
    Wa, sa, _ = make_w_q(N, K, seed=10)
    add("fallback_Wq_misaligned",
        "fallback: W_q 1 byte past a 16-byte boundary, x aligned: scalar "
        "kernel, bit-identical to qgemv_baseline",
        lambda: _fallback_check("fallback_Wq_misaligned", Wq_mis, scale, xa),
        expected="pass")
    add("fallback_x_misaligned",
        "fallback: x 2 bytes past a 16-byte boundary, W_q aligned: scalar "
        "kernel, bit-identical to qgemv_baseline",
        lambda: _fallback_check("fallback_x_misaligned", Wa, sa, xo_mis),
        expected="pass")
    Wk, sk, _ = make_w_q(16, 13, seed=11)
    xk = make_x_q(13, seed=12)
    add("fallback_K_not_mult16",
        "fallback: K = 13 (not a multiple of 16): scalar kernel, "
        "bit-identical to qgemv_baseline",
        lambda: _fallback_check("fallback_K_not_mult16", Wk, sk, xk),
        expected="pass")
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
                 "the vector contract (16-byte aligned W_q and x, K % 16 == "
                 "0) run the scalar kernel and are bit-identical to "
                 "qgemv_baseline"),
        "summary": summarize_cases(results),
        "cases": results,
    }
    if out_path is not None:
        out_path = Path(out_path)
        out_path.parent.mkdir(parents=True, exist_ok=True)
        out_path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
    return doc
