"""CPU tests of the command-line layer (cudalab_amd.cli, .regression,
.gen3): the reference CLI's subcommands and options parse
(scripts/cudalab.py:336-415), `benchmark winners` classifies saved matrix
records without a GPU, counter groups split into one pass each, and every
GPU command refuses cleanly when no GPU is visible."""
from __future__ import annotations

import json

import pytest

from cudalab_amd import cli, gen3, regression
from cudalab_amd.evaluator import experiment as E


def _parse(*argv):
    return cli.build_parser().parse_args(list(argv))


def test_subcommands_and_options_parse():
    a = _parse("test", "int4gemv", "--variant", "int4gemv_cdna4")
    assert (a.fn, a.op, a.variant, a.out_dir) == (cli.cmd_test, "int4gemv",
                                                  "int4gemv_cdna4", None)
    a = _parse("benchmark", "pair", "qgemv", "--parent", "qgemv_baseline",
               "--candidate", "qgemv_cdna4", "--M", "4096", "--H", "4096",
               "--tag", "t")
    assert a.fn is cli.cmd_bench_pair and (a.M, a.H) == (4096, 4096)
    assert (a.dtype, a.mode, a.rounds, a.caliber) == ("float16", "streaming", 9, "native")
    a = _parse("benchmark", "matrix", "gemv", "--variants", "gemv_cdna4,gemv_baseline",
               "--M", "1024", "--H", "4096", "--tag", "t", "--mode", "hot",
               "--dtype", "float32", "--caliber", "api")
    assert a.fn is cli.cmd_bench_matrix and (a.mode, a.dtype, a.caliber) == ("hot", "float32", "api")
    assert _parse("benchmark", "full", "int4gemv", "--tag", "t").fn is cli.cmd_bench_full
    assert _parse("benchmark", "winners", "int4gemv", "--tag", "t").fn is cli.cmd_bench_winners
    a = _parse("profile", "int4gemv", "--counters", "FETCH_SIZE;WRITE_SIZE",
               "--clock-control", "none")
    assert a.fn is cli.cmd_profile and (a.M, a.H, a.clock_control) == (4096, 4096, "none")
    assert _parse("pytorch", "qgemv", "--M", "8", "--H", "16").fn is cli.cmd_pytorch
    a = _parse("optimize", "int4gemv", "--id", "INT4GEMV-0001", "--parent", "int4gemv_lds_r2",
               "--candidate", "int4gemv_cdna4", "--hypothesis", "h", "--changes", "c",
               "--profile")
    assert a.fn is cli.cmd_optimize and a.profile and (a.M, a.H) == (4096, 4096)


@pytest.mark.parametrize("argv", [
    ["test", "softmax", "--variant", "x"],              # not a GEMV operator
    ["test", "int4gemv"],                               # --variant required
    ["benchmark", "pair", "int4gemv", "--parent", "a", "--candidate", "b",
     "--M", "8", "--H", "128"],                         # --tag required
    ["benchmark", "pair", "int4gemv", "--parent", "a", "--candidate", "b",
     "--M", "8", "--H", "128", "--tag", "t", "--caliber", "ncu"],
])
def test_bad_arguments_exit_2(argv):
    with pytest.raises(SystemExit) as e:
        _parse(*argv)
    assert e.value.code == 2


def test_counter_groups():
    assert cli._counter_groups(None) == []
    assert cli._counter_groups("FETCH_SIZE") == [["FETCH_SIZE"]]
    assert cli._counter_groups(" FETCH_SIZE ; WRITE_SIZE,GRBM_COUNT ;") == [
        ["FETCH_SIZE"], ["WRITE_SIZE", "GRBM_COUNT"]]


def _matrix_record(M, H, mode, ratio):
    return {"shape": [M, H], "dtype": "float16", "cache_mode": mode,
            "variants": ["a", "b"],
            "per_variant": {"a": {"median_us": 10.0}, "b": {"median_us": 10.0 * ratio}},
            "rounds": [{"valid": True, "us": {"a": 10.0, "b": 10.0 * ratio},
                        "us_raw": {"a": 10.0, "b": 10.0 * ratio}} for _ in range(9)]}


def test_benchmark_winners_from_saved_records(tmp_path, capsys):
    recs = {"t_M4096_H4096_float16_streaming": _matrix_record(4096, 4096, "streaming", 1.2),
            "t_M1024_H4096_float16_hot": _matrix_record(1024, 4096, "hot", 1.01)}
    for name, r in recs.items():
        (tmp_path / f"{name}.json").write_text(json.dumps(r))
    (tmp_path / "t_M1_H1_notes.json").write_text(json.dumps({"no": "per_variant"}))
    (tmp_path / "other_M8_H8_float16_hot.json").write_text(
        json.dumps(_matrix_record(8, 8, "hot", 2.0)))
    rc = cli.main(["benchmark", "winners", "int4gemv", "--tag", "t",
                   "--out-dir", str(tmp_path)])
    assert rc == 0
    doc = json.loads((tmp_path / "t_shape_winners.json").read_text())
    assert doc["operator"] == "int4gemv"
    cells = {(tuple(w["shape"]), w["cache_mode"]): w for w in doc["shape_winners"]}
    assert set(cells) == {((4096, 4096), "streaming"), ((1024, 4096), "hot")}
    assert cells[((4096, 4096), "streaming")]["status"] == E.SIGNIFICANT_WINNER
    assert cells[((1024, 4096), "hot")]["status"] == E.NO_UNIQUE_WINNER
    out = capsys.readouterr().out
    assert "winner=a" in out and "status=SIGNIFICANT_WINNER" in out


@pytest.mark.parametrize("argv", [
    ["test", "int4gemv", "--variant", "int4gemv_cdna4"],
    ["pytorch", "qgemv", "--M", "8", "--H", "16"],
    ["profile", "gemv"],
])
def test_gpu_commands_refuse_without_gpu(argv, monkeypatch, capsys):
    import torch
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert cli.main(argv) == 1
    assert "no GPU visible" in capsys.readouterr().err


def test_regression_and_gen3_refuse_without_gpu(monkeypatch, capsys, tmp_path):
    import torch
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert regression.main(["--out", str(tmp_path)]) == 1
    assert gen3.main(["--out", str(tmp_path)]) == 1
    assert regression.main(["--ops", "softmax"]) == 2
    err = capsys.readouterr().err
    assert "no GPU visible" in err and "--ops must name" in err


def test_gen3_uses_the_reference_variant_names():
    assert gen3.GENERATIONS == (("gemv", "gemv_vec4_row"), ("qgemv", "qgemv_vec16_row"),
                                ("int4gemv", "int4gemv_rowtile4_hx"))
    assert regression.OPS == ("int4gemv", "gemv", "qgemv")


def test_sweep_options(monkeypatch, capsys):
    """The sweep's --shapes / --modes / --variant options parse and reject
    malformed values before touching a GPU."""
    import torch
    from cudalab_amd.evaluator import sweep
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert sweep.main(["--shapes", "8192x28672,4096x4096"]) == 1     # parsed, no GPU
    assert sweep.main(["--variant", "int4gemv=int4gemv_cdna4,int4gemv_lds_tiled",
                       "--modes", "streaming"]) == 1
    assert sweep.main(["--modes", "misaligned,streaming"]) == 1
    for bad in (["--shapes", "8x8x8"], ["--shapes", "8xq"], ["--modes", "warm"],
                ["--variant", "softmax=x"], ["--variant", "int4gemv"], ["--ops", "rmsnorm"]):
        assert sweep.main(bad) == 2, bad
    err = capsys.readouterr().err
    assert "no GPU visible" in err and "--shapes" in err


def test_sweep_misaligned_sets_keep_values_off_alignment():
    """The misaligned mode's copies hold the same values at a base address
    1 (W) or 2 (x) bytes past a 16-byte boundary."""
    import torch
    from cudalab_amd.evaluator.sweep import offset_copy
    for dtype, off in ((torch.uint8, 1), (torch.int8, 1), (torch.float16, 2)):
        t = torch.arange(48).to(dtype).view(3, 16)
        v = offset_copy(t, off)
        assert v.data_ptr() % 16 == off and v.is_contiguous()
        assert torch.equal(v, t) and v.shape == t.shape and v.dtype == dtype


def test_decode_stress_option(monkeypatch, capsys):
    """--stress is parsed and needs a GPU; the sequence is the 7B MLP pair,
    then four 4096^2 projections."""
    import torch
    from cudalab_amd import decode
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert decode.main(["--stress", "--op", "qgemv"]) == 1
    assert "no GPU visible" in capsys.readouterr().err
    assert decode.STRESS_SHAPES == ((11008, 4096), (4096, 11008)) + ((4096, 4096),) * 4


def test_timeline_options(monkeypatch, capsys):
    """The timeline command rejects impossible sizes before touching a GPU
    and needs one to run."""
    import torch
    from cudalab_amd.evaluator import timeline
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert timeline.main(["--n", "4096", "--k", "11008"]) == 1
    for bad in (["--launches", "1"], ["--k", "100"], ["--n", "0"]):
        assert timeline.main(bad) == 2, bad
    err = capsys.readouterr().err
    assert "no GPU visible" in err and "multiple of 128" in err
