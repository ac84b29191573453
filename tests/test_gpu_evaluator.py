"""GPU tests of the A/B engine (evaluator.bench: measure_block, bench_pair,
bench_matrix) on the real INT4 path: records are complete, the round
structure holds, and the fixed decision rules apply to what was measured.
Short settings (5 rounds, 60 samples of 8 launches) keep each test to
seconds; the verdicts themselves are not asserted (they depend on the
hardware), only that they are well formed."""
from __future__ import annotations

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

FAST = dict(rounds=5, warmup=16, iters=60, batch=8)


@pytest.fixture(scope="module")
def op4(ext4):
    from cudalab_amd.operators import get
    return get("int4gemv")


def test_measure_block_both_calibers(op4, ext4):
    import torch
    from cudalab_amd.evaluator.bench import measure_block
    for mode in ("streaming", "hot"):
        pool = op4.make_bench_pool(1024, 4096, torch.float16, mode)
        for caliber in ("native", "api"):
            announce(f"measure_block {mode} {caliber}")
            b = measure_block(pool, ext4, "int4gemv_cdna4", warmup=16, iters=60,
                              batch=8, warmup_ms=50.0, caliber=caliber)
            assert b["n_raw"] == 60 and b["caliber"] == caliber
            assert b["n_accepted"] + b["n_rejected_fast"] + b["n_rejected_slow"] == 60
            assert 0 < b["min_us"] <= b["raw_median_us"]
            assert b["median_us"] > 0
        del pool


def test_bench_pair_record(op4, ext4):
    from cudalab_amd.evaluator.ab import decide_pair
    from cudalab_amd.evaluator.bench import bench_pair
    from cudalab_amd.evaluator import decision as D
    announce("bench_pair int4gemv_wave_r2 -> int4gemv_cdna4 1024x4096 streaming")
    rec = bench_pair(op4, ext4, "int4gemv_wave_r2", "int4gemv_cdna4", 1024, 4096,
                     mode="streaming", **FAST)
    assert rec["n_rounds"] == 5 and len(rec["rounds"]) == 5
    assert [r["order"][0] for r in rec["rounds"]] == \
        ["int4gemv_wave_r2", "int4gemv_cdna4"] * 2 + ["int4gemv_wave_r2"]
    assert len(rec["speedups"]) == rec["valid_rounds"]
    assert all(s > 0 for s in rec["speedups"])
    assert rec["pool"]["working_set_gt_llc"] and rec["pool"]["pool_extra"]["hbm_cold"]
    v = decide_pair(rec, True)
    assert v["policy_decision"] in (D.KEEP, D.REJECT, D.NEUTRAL, D.UNSTABLE)
    assert v["statistical_relation"] in (D.FASTER, D.SLOWER, D.UNRESOLVED)
    assert rec["gpu_state_before"] is not None and rec["gpu_state_after"] is not None


def test_bench_matrix_cell(op4, ext4):
    import torch
    from cudalab_amd.evaluator.bench import analyze_shape_winners, bench_matrix
    variants = ["int4gemv_cdna4", "int4gemv_lds_r1", "int4gemv_wave_r2"]
    announce("bench_matrix int4gemv 1024x4096 hot")
    rec = bench_matrix(op4, ext4, variants, 1024, 4096, dtype=torch.float16,
                       mode="hot", **FAST)
    assert [r["order"][0] for r in rec["rounds"]] == variants + variants[:2]
    [cell] = analyze_shape_winners([rec])
    assert cell["winner"] in variants and cell["runner_up"] in variants
    assert set(rec["per_variant"]) == set(variants)
    with pytest.raises(ValueError, match="unknown variant"):
        bench_matrix(op4, ext4, ["int4gemv_cdna4", "no_such"], 64, 128, **FAST)


def test_launch_floor_and_read_ceiling(ext4):
    """The two reference points the bench reports beside a GEMV call: the
    empty-launch floor of the GEMV's launch shape, and the plain read of the
    same bytes.  A read does strictly more than an empty launch, so its time
    per call is the larger; both are small positive numbers."""
    from cudalab_amd import ext as E
    announce("launch_floor 256x512")
    floor = E.launch_floor(256, 512, warmup=50, n_launches=500)
    announce("read_ceiling 8667136 B")
    ceil = E.read_ceiling(8667136, warmup=50, n_launches=500)
    assert 0 < floor < 50.0
    assert 0 < ceil["us_per_call"] < 50.0
    assert floor < 2 * ceil["us_per_call"]
    for grid, block in ((0, 256), (256, 0), (256, 1025)):
        with pytest.raises(RuntimeError, match="grid must be"):
            E.launch_floor(grid, block, warmup=0, n_launches=1)


def test_api_cost_paths_all_launch(cuda):
    """The host-cost tool times real launches on every path: each raw entry
    point is status-checked before and after, and no path can read below
    the cost of an enqueue (a refused call returns in ~0.1 us)."""
    from cudalab_amd.evaluator import api_cost
    res = api_cost.run(n=1024, k=1024, calls=50, reps=2)
    floor = res["native_enqueue_us_per_launch"]
    assert floor > 0.5
    for name, rec in res["host_us_per_call"].items():
        assert rec["us"] is not None and rec["samples"] == 2, name
        assert rec["us"] > 0.5 * floor, (name, rec, floor)


@pytest.mark.parametrize("N,K", [(4096, 4096), (11008, 4096), (4096, 11008), (300, 1280)])
def test_timeline_stamps_every_wave_and_keeps_the_outputs(ext4, N, K):
    """cq_int4_timeline runs a stamped copy of the LDS kernel: every wave of
    every timed launch leaves five stamps in order (start <= x barrier <=
    first chunk <= last chunk <= y stored), the launches follow one another,
    and each set's y is bit-identical to forward_into's (the copy keeps the
    product kernel's arithmetic).  Plans covered: one row per lane on 512
    threads, two rows per lane on 256, six chunks per lane, a short row."""
    import numpy as np
    import torch
    from cudalab_amd.evaluator.timeline import by_workgroup, run_stamped, summarize
    from cudalab_amd.operators.int4gemv import device_random_set
    sets = [device_random_set(N, K, 900 + i) for i in range(3)]
    announce(f"timeline {N}x{K}")
    r = run_stamped("int4gemv_cdna4", sets, n_launches=6, warmup=3, burn_ms=0.0,
                    delay_us=2000.0)
    a = r["stamps"]
    d = ext4.describe("int4gemv_cdna4", sets[0][0], sets[0][2])
    assert a.shape == (6, int(d["grid"]) * int(d["block"]) // 64, 8)
    t = a[:, :, :5]
    assert (t > 0).all()
    assert (np.diff(t, axis=2) >= 0).all()
    starts = t[:, :, 0].min(axis=1)
    ends = t[:, :, 4].max(axis=1)
    assert (starts[1:] >= ends[:-1] - 5).all()    # one stream: launches in order (50 ns slack)
    s = summarize(a, r["ticks_per_us"], skip=0.0)
    assert s["launches_used"] == 5 and 0 < s["span_us"] < 1000
    g = by_workgroup(a, r["ticks_per_us"], int(d["block"]) // 64, skip=0.0)
    assert g["workgroups"] == int(d["grid"]) and g["launches_used"] == 6
    assert 0 < g["barrier_first_on_cu_us"] < 1000
    if g["barrier_second_on_cu_us"] is not None:      # a CU held two workgroups
        assert 0 < g["barrier_second_on_cu_us"] < 1000
    assert 1 <= len(g["barrier_by_xcd_us"]) <= 8
    for W, sc, x, out in sets:
        want = torch.empty_like(out)
        ext4.forward_into("int4gemv_cdna4", W, sc, x, want)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
