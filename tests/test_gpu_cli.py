"""GPU tests of the command-line layer on the real path: `test`,
`benchmark pair`, `optimize` and `pytorch` of cudalab_amd.cli (the
reference's scripts/cudalab.py commands), the regression over all normal
variants (scripts/regression_v07.py) and the three-generation native
timing (scripts/gen3_native_timing.py).  Benchmarks use hot pools and 5
rounds to stay short; verdicts depend on the hardware and are only checked
for form."""
from __future__ import annotations

import json

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def test_cli_test_passes_and_gates(cuda, tmp_path, capsys):
    from cudalab_amd import cli
    announce("cli test int4gemv --variant int4gemv_cdna4")
    rc = cli.main(["test", "int4gemv", "--variant", "int4gemv_cdna4",
                   "--out-dir", str(tmp_path), "--neg-out-dir", str(tmp_path)])
    out = capsys.readouterr().out
    assert rc == 0, out
    assert "[correctness] int4gemv_cdna4: all_pass=True" in out
    assert "[negative] all_pass=True" in out
    assert (tmp_path / "int4gemv_cdna4.json").exists()
    announce("cli test qgemv via a reference alias")
    assert cli.main(["test", "qgemv", "--variant", "qgemv_vec16_row",
                     "--out-dir", str(tmp_path), "--neg-out-dir", str(tmp_path)]) == 0
    announce("cli gates: unknown and quarantined variants")
    assert cli.main(["test", "int4gemv", "--variant", "int4gemv_nope"]) == 2
    assert "未知变体 'int4gemv_nope'" in capsys.readouterr().err
    assert cli.main(["test", "gemv", "--variant", "gemv_splitk4"]) == 2
    assert "已被隔离" in capsys.readouterr().err


def test_cli_benchmark_pair_and_optimize(cuda, tmp_path, capsys):
    from cudalab_amd import cli
    from cudalab_amd.operators import get
    announce("cli benchmark pair int4gemv 1024x4096 hot, 5 rounds")
    rc = cli.main(["benchmark", "pair", "int4gemv", "--parent", "int4gemv_lds_r1",
                   "--candidate", "int4gemv_cdna4", "--M", "1024", "--H", "4096",
                   "--mode", "hot", "--rounds", "5", "--tag", "pair_t",
                   "--out-dir", str(tmp_path)])
    assert rc == 0
    rec = json.loads((tmp_path / "pair_t.json").read_text())
    assert rec["n_rounds"] == 5 and rec["parent"] == "int4gemv_lds_r1"
    assert "[pair] int4gemv_lds_r1 vs int4gemv_cdna4" in capsys.readouterr().out
    op = get("qgemv")
    before = set(op.experiments_dir.glob("*.json")) if op.experiments_dir.exists() else set()
    announce("cli optimize qgemv 1024x4096 hot, 5 rounds")
    rc = cli.main(["optimize", "qgemv", "--id", "QGEMV-TEST", "--parent", "qgemv_lds_r2",
                   "--candidate", "qgemv_cdna4", "--hypothesis", "h", "--changes", "c",
                   "--M", "1024", "--H", "4096", "--mode", "hot", "--rounds", "5"])
    out = capsys.readouterr().out
    assert rc == 0, out
    assert "== [QGEMV-TEST] decision:" in out and "statistical_relation:" in out
    new = set(op.experiments_dir.glob("*.json")) - before
    doc = json.loads((op.experiments_dir / "QGEMV-TEST.json").read_text())
    assert op.experiments_dir / "QGEMV-TEST.json" in new
    assert doc["decision"]["policy_decision"] in ("KEEP", "REJECT", "NEUTRAL", "UNSTABLE")
    assert doc["correctness"]["all_pass"] and doc["negative"]["all_pass"]
    assert doc["paired_benchmark"]["paired_rounds"] == 5


def test_cli_pytorch_context(cuda, capsys):
    from cudalab_amd import cli
    announce("cli pytorch int4gemv 1024x4096")
    assert cli.main(["pytorch", "int4gemv", "--M", "1024", "--H", "4096"]) == 0
    out = capsys.readouterr().out
    d = json.loads(out[out.index("{"):])
    assert d["available"] and d["median_us"] > 0


def test_regression_gemv(cuda, tmp_path, capsys):
    from cudalab_amd import regression
    announce("regression --ops gemv")
    assert regression.main(["--out", str(tmp_path), "--ops", "gemv"]) == 0
    assert capsys.readouterr().out.rstrip().endswith("SUMMARY all_pass")
    audit = json.loads((tmp_path / "quarantine_audit.json").read_text())
    assert audit["gemv"]["quarantined_variants()"] == ["gemv_splitk4"]
    assert "gemv_splitk4" not in audit["gemv"]["variants()"]
    summary = json.loads((tmp_path / "summary.json").read_text())
    assert set(summary["gemv"]["variants_run"]) == {"gemv_baseline", "gemv_cdna4",
                                                    "gemv_lds_tiled"}


def test_gen3_native_timing(cuda, tmp_path, capsys):
    from cudalab_amd import gen3
    announce("gen3 native timing 4096x4096 (FP16, INT8, INT4)")
    assert gen3.main(["--out", str(tmp_path)]) == 0
    for op, variant in gen3.GENERATIONS:
        doc = json.loads((tmp_path / op / f"native_timing_{variant}_4096.json").read_text())
        assert doc["resolves_to"].endswith("_cdna4")
        for tag in ("w200", "w5000"):
            assert doc[tag]["median_us"] > 0 and doc[tag]["n_windows"] == 10
