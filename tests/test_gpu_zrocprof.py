"""GPU test of the rocprofv3 adapter (evaluator.profiler.profile_variant):
the operator's driver runs under `rocprofv3 --kernel-trace` in a child
process, and a separate `--pmc` pass reads FETCH_SIZE; the summary names
the INT4 kernel with device durations and the counter.  Collected late
(file name) because it starts child processes."""
from __future__ import annotations

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def test_profile_variant(cuda, tmp_path):
    from cudalab_amd.evaluator.profiler import profile_variant, rocprof_path
    from cudalab_amd.operators import get
    if rocprof_path() is None:
        pytest.skip("rocprofv3 not installed")
    announce("profile_variant int4gemv_cdna4 1024x4096 (trace + FETCH_SIZE pass)")
    s = profile_variant(get("int4gemv"), "int4gemv_cdna4", 1024, 4096,
                        out_dir=tmp_path, counters=[["FETCH_SIZE"]], timeout=240)
    assert s["kernels"], s["errors"]
    k = s["kernels"][0]
    assert "int4gemv" in k["name"] and k["n"] >= 6 and k["median_us"] > 0
    assert s["kernel_duration_us"] == k["median_us"]
    assert s["algorithmic_bw_gbps"] > 0
    assert s["counters"]["FETCH_SIZE"] is not None and s["counters"]["FETCH_SIZE"] > 0
    assert (tmp_path / "summary.json").exists()


def test_cli_profile(cuda, tmp_path, capsys):
    from cudalab_amd import cli
    from cudalab_amd.evaluator.profiler import rocprof_path
    if rocprof_path() is None:
        pytest.skip("rocprofv3 not installed")
    announce("cli profile qgemv --variants qgemv_cdna4 1024x4096 --counters FETCH_SIZE")
    rc = cli.main(["profile", "qgemv", "--variants", "qgemv_cdna4", "--M", "1024",
                   "--H", "4096", "--counters", "FETCH_SIZE", "--out-dir", str(tmp_path)])
    assert rc == 0
    import json
    s = json.loads((tmp_path / "qgemv_cdna4_M1024_H4096" / "summary.json").read_text())
    assert s["kernels"] and s["kernel_duration_us"] > 0, s["errors"]
    assert s["counters"]["FETCH_SIZE"] and s["clock_control"]["applied"] is False
    assert "duration=" in capsys.readouterr().out
