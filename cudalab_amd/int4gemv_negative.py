"""INT4 W4A16 GEMV negative suite (per variant).

Drop-in for `cudalab/int4gemv_negative.py:71-347`: illegal inputs must be
rejected before any launch with an explicit message; legal inputs must never
be rejected; inputs that miss the vector contract (16-byte aligned W_packed
and x, K % 32 == 0) must run the scalar kernel and be bit-identical to
`int4gemv_baseline`.  After every case a control forward checks that the
device context is healthy.

Cases (the reference's 30 plus one):
  W_packed 8: 1d / 3d / N_zero / K2_zero / dtype_fp16 / dtype_int8 / cpu /
              noncontig
  K        1: K_not_mult128 (hard reject, before the scale checks)
  scale    6: group_count / N_mismatch / 1d / dtype_fp32 / cpu / noncontig
  x        5: len_mismatch / 2d / dtype_fp32 / cpu / noncontig
  out      4: wrong_shape / wrong_dtype / noncontig / cpu
  variant  1: unknown_variant
  control  3: valid_forward_into_control / valid_offset_view_Wp_control /
              valid_offset_view_x_control
  fallback 3: fallback_Wp_misaligned (W +1 B) / fallback_x_misaligned
              (x +2 B) / fallback_Wp_x_misaligned (W +2 B and x +2 B
              together, the misaligned configuration of the benchmark spec)
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from .evaluator.gpu import now_iso
from .evaluator.negative import run_case, summarize_cases
from .operators.int4gemv import make_w4, make_x4

SUITE_VERSION = "negative-int4gemv"
V = "int4gemv_baseline"


def _post_check_ok(ext, variant: str = V) -> bool:
    try:
        torch.cuda.synchronize()
        W_packed, scale, _ = make_w4(2, 128, seed=0)
        x = make_x4(128, seed=1)
        y = ext.forward(variant, W_packed, scale, x)
        torch.cuda.synchronize()
        return bool(torch.isfinite(y.float()).all())
    except Exception:  # noqa: BLE001
        return False


def _rand_bytes(shape, seed: int, device: str = "cuda") -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(0, 256, shape, generator=g, dtype=torch.uint8).to(device)


def _offset_view(src: torch.Tensor, offset: int, shape) -> torch.Tensor:
    """Contiguous view of `shape` starting `offset` elements into src."""
    n = 1
    for d in shape:
        n *= d
    return src[offset:offset + n].view(*shape)


def build_cases(ext, variant: str = V) -> list[dict]:
    dev = "cuda"
    cases: list[dict] = []

    def add(cid, description, call, expected="reject",
            expect_msg_contains=None):
        cases.append(dict(id=cid, variant=variant, description=description,
                          call=call, expected=expected,
                          expect_msg_contains=expect_msg_contains))

    N, K = 8, 256
    W_packed, scale, _ = make_w4(N, K, seed=0)
    x = make_x4(K, seed=1)

    def fwd(Wa, sa, xa):
        return ext.forward(variant, Wa, sa, xa)

    # ---- W_packed ----
    w_1d = _rand_bytes((N * K // 2,), 2)
    add("W_packed_1d", "W_packed is 1-D (N*K/2,)",
        lambda: fwd(w_1d, scale, x), expect_msg_contains="必须是 2 维")
    w_3d = _rand_bytes((N, K // 2), 3).view(2, N // 2, K // 2)
    add("W_packed_3d", "W_packed is 3-D (2, 4, K/2)",
        lambda: fwd(w_3d, scale, x), expect_msg_contains="必须是 2 维")
    w_n0 = torch.empty(0, K // 2, dtype=torch.uint8, device=dev)
    add("W_packed_N_zero", "N = 0",
        lambda: fwd(w_n0, scale[:0].contiguous(), x),
        expect_msg_contains="N 必须 > 0")
    w_k0 = torch.empty(N, 0, dtype=torch.uint8, device=dev)
    add("W_packed_K2_zero", "K/2 = 0",
        lambda: fwd(w_k0, scale, x), expect_msg_contains="K/2 必须 > 0")
    w_f16 = torch.randn(N, K // 2, dtype=torch.float16, device=dev)
    add("W_packed_dtype_fp16", "W_packed is fp16 (must be uint8)",
        lambda: fwd(w_f16, scale, x), expect_msg_contains="必须是 uint8")
    w_i8 = _rand_bytes((N, K // 2), 12).to(torch.int8)
    add("W_packed_dtype_int8", "W_packed is int8 (must be uint8)",
        lambda: fwd(w_i8, scale, x), expect_msg_contains="必须是 uint8")
    w_cpu = _rand_bytes((N, K // 2), 4, device="cpu")
    add("W_packed_cpu", "W_packed on the CPU",
        lambda: fwd(w_cpu, scale.cpu(), x.cpu()),
        expect_msg_contains="CUDA 张量")
    w_t = _rand_bytes((K, N // 2), 5).t()
    add("W_packed_noncontig", "W_packed is a transposed (non-contiguous) view",
        lambda: fwd(w_t, scale, x), expect_msg_contains="连续内存")

    # ---- K % 128: hard reject, checked before the scale checks ----
    w_k64 = _rand_bytes((N, 32), 6)
    add("K_not_mult128", "K = 64 is not a multiple of 128",
        lambda: fwd(w_k64, torch.zeros(N, 1, dtype=torch.float16, device=dev),
                    make_x4(64, seed=6)),
        expect_msg_contains="必须可被 128 整除")

    # ---- scale ----
    s_short = scale[:, :scale.size(1) - 1].contiguous()
    add("scale_group_count", "scale has K/128 - 1 groups (invalid group count)",
        lambda: fwd(W_packed, s_short, x),
        expect_msg_contains="scale 组数必须等于 K/128")
    s_nshort = scale[:N - 1].contiguous()
    add("scale_N_mismatch", "scale has N - 1 rows",
        lambda: fwd(W_packed, s_nshort, x),
        expect_msg_contains="scale 行数必须等于 N")
    s_1d = scale.view(N * (K // 128))
    add("scale_1d", "scale is 1-D",
        lambda: fwd(W_packed, s_1d, x), expect_msg_contains="必须是 2 维")
    s_f32 = scale.float()
    add("scale_dtype_fp32", "scale is fp32 (must be fp16)",
        lambda: fwd(W_packed, s_f32, x), expect_msg_contains="必须是 float16")
    add("scale_cpu", "scale on the CPU, W_packed on the GPU",
        lambda: fwd(W_packed, scale.cpu(), x), expect_msg_contains="CUDA 张量")
    s_big = torch.randn(2 * N, scale.size(1), dtype=torch.float16, device=dev)
    s_nc = s_big[::2]
    add("scale_noncontig", "scale is a stride-2 row slice",
        lambda: fwd(W_packed, s_nc, x), expect_msg_contains="连续内存")

    # ---- x ----
    x_short = make_x4(K - 128, seed=7)
    add("x_len_mismatch", "x has K - 128 elements",
        lambda: fwd(W_packed, scale, x_short),
        expect_msg_contains="x 长度必须等于 K")
    x_2d = x.view(1, K)
    add("x_2d", "x is 2-D (1, K)",
        lambda: fwd(W_packed, scale, x_2d), expect_msg_contains="必须是 1 维")
    x_f32 = make_x4(K, seed=8).float()
    add("x_dtype_fp32", "x is fp32 (must be fp16)",
        lambda: fwd(W_packed, scale, x_f32), expect_msg_contains="必须是 float16")
    add("x_cpu", "x on the CPU, W_packed on the GPU",
        lambda: fwd(W_packed, scale, x.cpu()), expect_msg_contains="CUDA 张量")
    x_big = torch.randn(2 * K, dtype=torch.float16, device=dev)
    x_nc = x_big[::2]
    add("x_noncontig", "x is a stride-2 slice",
        lambda: fwd(W_packed, scale, x_nc), expect_msg_contains="连续内存")

    # ---- out of forward_into ----
    add("out_wrong_shape", "out has N - 1 elements",
        lambda: ext.forward_into(variant, W_packed, scale, x,
                                 torch.empty(N - 1, dtype=torch.float16,
                                             device=dev)),
        expect_msg_contains="out 长度必须等于 N")
    add("out_wrong_dtype", "out is fp32 (must be fp16)",
        lambda: ext.forward_into(variant, W_packed, scale, x,
                                 torch.empty(N, dtype=torch.float32,
                                             device=dev)),
        expect_msg_contains="必须是 float16")
    o_big = torch.randn(2 * N, dtype=torch.float16, device=dev)
    o_nc = o_big[::2]
    add("out_noncontig", "out is a stride-2 slice",
        lambda: ext.forward_into(variant, W_packed, scale, x, o_nc),
        expect_msg_contains="连续内存")
    add("out_cpu", "out on the CPU",
        lambda: ext.forward_into(variant, W_packed, scale, x,
                                 torch.empty(N, dtype=torch.float16)),
        expect_msg_contains="CUDA 张量")

    # ---- variant name ----
    add("unknown_variant", "unknown variant name (registry lookup)",
        lambda: ext.forward("no_such_int4gemv_variant", W_packed, scale, x),
        expect_msg_contains="未知 int4gemv 变体")

    # ---- controls: legal inputs are never rejected ----
    out_ok = torch.empty(N, dtype=torch.float16, device=dev)
    add("valid_forward_into_control", "control: legal forward_into succeeds",
        lambda: ext.forward_into(variant, W_packed, scale, x, out_ok),
        expected="pass")
    big_wp = _rand_bytes((N * K // 2 + 16,), 9)
    Wp_mis = _offset_view(big_wp, 1, (N, K // 2))    # base + 1 byte

    def _wp_offset_control():
        ext.forward_into(variant, Wp_mis, scale, x, out_ok)
        y = ext.forward(variant, W_packed, scale, x)
        assert torch.isfinite(out_ok.float()).all(), "offset-view output not finite"
        assert torch.isfinite(y.float()).all(), "control output not finite"

    add("valid_offset_view_Wp_control",
        "control: W_packed is a contiguous view 1 byte past a 16-byte "
        "boundary; legal, must succeed", _wp_offset_control, expected="pass")
    big_x = torch.randn(K + 8, dtype=torch.float16, device=dev)
    x_mis = _offset_view(big_x, 1, (K,))              # base + 2 bytes
    add("valid_offset_view_x_control",
        "control: x is a contiguous slice 2 bytes past a 16-byte boundary; "
        "legal, must succeed",
        lambda: fwd(W_packed, scale, x_mis), expected="pass")

    # ---- fallback: bit-identical to int4gemv_baseline ----
    def _fallback_check(cid, Wm, sm, xm):
        out_f = torch.empty(Wm.size(0), dtype=torch.float16, device=dev)
        ext.forward_into(variant, Wm, sm, xm, out_f)
        torch.cuda.synchronize()
        y_base = ext.forward("int4gemv_baseline", Wm, sm, xm)
        torch.cuda.synchronize()
        assert torch.equal(out_f, y_base), (
            f"{cid}: fallback output differs from int4gemv_baseline (must be "
            "bit-identical: same scalar kernel)")

    xa = make_x4(K, seed=10)
    Wa, sa, _ = make_w4(N, K, seed=11)
    add("fallback_Wp_misaligned",
        "fallback: W_packed 1 byte past a 16-byte boundary, x aligned: "
        "scalar kernel, bit-identical to int4gemv_baseline",
        lambda: _fallback_check("fallback_Wp_misaligned", Wp_mis, scale, xa),
        expected="pass")
    add("fallback_x_misaligned",
        "fallback: x 2 bytes past a 16-byte boundary, W_packed aligned: "
        "scalar kernel, bit-identical to int4gemv_baseline",
        lambda: _fallback_check("fallback_x_misaligned", Wa, sa, x_mis),
        expected="pass")
    big_wa = torch.zeros(N * K // 2 + 16, dtype=torch.uint8, device=dev)
    Wa2 = _offset_view(big_wa, 2, (N, K // 2))        # base + 2 bytes
    Wa2.copy_(Wa)
    add("fallback_Wp_x_misaligned",
        "fallback: W_packed and x both 2 bytes past a 16-byte boundary: "
        "scalar kernel, bit-identical to int4gemv_baseline",
        lambda: _fallback_check("fallback_Wp_x_misaligned", Wa2, sa, x_mis),
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
        "note": ("illegal inputs are rejected before launch; K % 128 != 0 is "
                 "a hard reject; inputs missing the vector contract (16-byte "
                 "aligned W_packed and x, K % 32 == 0) run the scalar kernel "
                 "and are bit-identical to int4gemv_baseline"),
        "summary": summarize_cases(results),
        "cases": results,
    }
    if out_path is not None:
        out_path = Path(out_path)
        out_path.parent.mkdir(parents=True, exist_ok=True)
        out_path.write_text(json.dumps(doc, indent=2, ensure_ascii=False))
    return doc
