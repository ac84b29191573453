"""Short text summaries of rocprofv3 output directories.

Three reports, all printed to stdout:

  trace    per-kernel dispatch durations from a `--kernel-trace --stats` run
           (count, mean, median, min, max, and the median gap between
           consecutive dispatches of the same kernel); optionally the
           matched kernel's figures as JSON for bench.py's
           `rocprof_isolated_dispatch_us` field
  counters per-dispatch medians of every counter in one or more `--pmc`
           runs, for the kernels matching each --match string
  traffic  HBM bytes per dispatch of one kernel from two `--pmc` runs
           (FETCH_SIZE, then WRITE_SIZE), each scaled by what the same
           counter reads for a calibration copy of known size in the same
           run; optionally written as JSON for bench.py's `traffic` field

Reads rocprofv3's CSV output (`-f csv`: *_kernel_trace.csv,
*_kernel_stats.csv, *_counter_collection.csv) or its SQLite database
(the default rocpd format: views `kernels` and `counters_collection`).

Usage:
  python -m cudalab_amd.evaluator.rocprof_summary trace DIR [--match S]
      [--top N] [--by-grid] [--shape N K --json-out FILE [--after K2]]
  python -m cudalab_amd.evaluator.rocprof_summary counters DIR [DIR ...]
      --match S [--match S ...]
  python -m cudalab_amd.evaluator.rocprof_summary traffic --fetch DIR
      --write DIR --match S --calib-match S --calib-bytes B
      [--shape N K] [--json-out FILE]
"""
from __future__ import annotations

import argparse
import csv
import json
import sqlite3
import statistics
import sys
from pathlib import Path


def _col(header: list[str], *names: str) -> int:
    low = [h.strip().lower() for h in header]
    for n in names:
        if n.lower() in low:
            return low.index(n.lower())
    raise KeyError(f"none of {names} in CSV header {header}")


def _csv_rows(d: Path, suffix: str) -> list[tuple[list[str], list[list[str]]]]:
    out = []
    for f in sorted(d.rglob(f"*{suffix}")):
        with open(f, newline="") as fh:
            r = list(csv.reader(fh))
        if r:
            out.append((r[0], r[1:]))
    return out


def _dbs(d: Path) -> list[Path]:
    return sorted(d.rglob("*.db"))


def dispatch_times(d: Path, by_grid: bool = False) -> dict[str, list[tuple[int, int]]]:
    """kernel name -> [(start_ns, end_ns)] in start order.  With `by_grid`
    the key also carries the dispatch's grid size (CSV traces), so one
    kernel launched at several shapes is reported per shape."""
    by: dict[str, list[tuple[int, int]]] = {}
    tables = _csv_rows(d, "kernel_trace.csv")
    for header, rows in tables:
        ni = _col(header, "Kernel_Name", "Name")
        si = _col(header, "Start_Timestamp", "Start")
        ei = _col(header, "End_Timestamp", "End")
        gi = None
        if by_grid:
            try:
                gi = _col(header, "Grid_Size_X", "Grid_Size", "Grid_SizeX")
            except KeyError:
                gi = None
        for r in rows:
            key = r[ni] if gi is None else f"{r[ni]} [grid={r[gi]}]"
            by.setdefault(key, []).append((int(r[si]), int(r[ei])))
    if not tables:
        for db in _dbs(d):
            con = sqlite3.connect(db)
            for n, s, e in con.execute("select name, start, end from kernels"):
                by.setdefault(n, []).append((int(s), int(e)))
            con.close()
    for v in by.values():
        v.sort()
    return by


def counter_names(d: Path) -> list[str]:
    names: set[str] = set()
    tables = _csv_rows(d, "counter_collection.csv")
    for header, rows in tables:
        ci = _col(header, "Counter_Name")
        names.update(r[ci] for r in rows)
    if not tables:
        for db in _dbs(d):
            con = sqlite3.connect(db)
            names.update(r[0] for r in con.execute(
                "select distinct counter_name from counters_collection"))
            con.close()
    return sorted(names)


def counter_values(d: Path, counter: str) -> dict[str, list[float]]:
    """kernel name -> per-dispatch values of `counter`."""
    by: dict[str, list[float]] = {}
    tables = _csv_rows(d, "counter_collection.csv")
    for header, rows in tables:
        ni = _col(header, "Kernel_Name", "Name")
        ci = _col(header, "Counter_Name")
        vi = _col(header, "Counter_Value", "Value")
        di = None
        try:
            di = _col(header, "Dispatch_Id")
        except KeyError:
            pass
        acc: dict[tuple, float] = {}
        for i, r in enumerate(rows):
            if r[ci] != counter:
                continue
            key = (r[ni], r[di] if di is not None else i)
            acc[key] = acc.get(key, 0.0) + float(r[vi])
        for (n, _), v in acc.items():
            by.setdefault(n, []).append(v)
    if not tables:
        for db in _dbs(d):
            con = sqlite3.connect(db)
            cols = [r[1] for r in con.execute("pragma table_info(counters_collection)")]
            name = "kernel_name" if "kernel_name" in cols else "name"
            val = "value" if "value" in cols else "counter_value"
            disp = "dispatch_id" if "dispatch_id" in cols else "rowid"
            q = (f"select {name}, {disp}, sum({val}) from counters_collection "
                 f"where counter_name = ? group by {name}, {disp}")
            for n, _, v in con.execute(q, (counter,)):
                by.setdefault(n, []).append(float(v))
            con.close()
    return by


def _pick(by: dict, match: str) -> tuple[str, list]:
    hits = [k for k in by if match in k]
    if not hits:
        raise SystemExit(f"no kernel matching {match!r}; have: "
                         + "; ".join(k[:80] for k in by))
    best = max(hits, key=lambda k: len(by[k]))
    return best, by[best]


def _stats_us(ns: list[float]) -> dict:
    s = sorted(ns)
    return {"n": len(s), "mean": statistics.fmean(s) / 1e3,
            "median": s[len(s) // 2] / 1e3, "min": s[0] / 1e3,
            "max": s[-1] / 1e3}


def report_trace(d: Path, match: str | None, top: int = 8,
                 by_grid: bool = False) -> str:
    by = dispatch_times(d, by_grid)
    rows = []
    for name, v in by.items():
        st = _stats_us([e - s for s, e in v])
        gaps = sorted(v[i + 1][0] - v[i][1] for i in range(len(v) - 1)) or [0]
        st["gap_median"] = gaps[len(gaps) // 2] / 1e3
        st["total"] = st["mean"] * st["n"]
        rows.append((name, st))
    rows.sort(key=lambda r: -r[1]["total"])
    lines = [f"{'kernel':<72} {'n':>6} {'mean_us':>9} {'median':>9} "
             f"{'min':>8} {'max':>9} {'gap_med':>8}"]
    chosen = [r for r in rows if match and match in r[0]]
    for name, st in (chosen + [r for r in rows if r not in chosen])[:top]:
        if "[grid=" in name and len(name) > 72:      # keep the grid visible
            head, grid = name.rsplit(" [grid=", 1)
            name = head[:72 - len(grid) - 8] + " [grid=" + grid
        lines.append(f"{name[:72]:<72} {st['n']:>6} {st['mean']:>9.3f} "
                     f"{st['median']:>9.3f} {st['min']:>8.3f} {st['max']:>9.3f} "
                     f"{st['gap_median']:>8.3f}")
    stats = _csv_rows(d, "kernel_stats.csv")
    for header, srows in stats:
        ni = _col(header, "Name")
        ai = _col(header, "AverageNs")
        ci = _col(header, "Calls")
        lines.append("")
        lines.append("rocprofv3 --stats (kernel_stats.csv):")
        for r in srows[:top]:
            lines.append(f"  {r[ni][:72]:<72} calls={r[ci]:>6} "
                         f"avg_us={float(r[ai]) / 1e3:.3f}")
    return "\n".join(lines)


def trace_record(d: Path, match: str, after: str | None = None) -> dict:
    """The dispatch-duration figures of the kernel matching `match` (the
    one with the most dispatches).  With `after`, only its dispatches that
    start after the end of the last dispatch of the kernel matching `after`
    count (bench.py queues an on-device wait right before its timed window,
    so `after="delay_kernel"` selects the window), and the record also gives
    the window's start-to-start rate: (last end - first start) / n."""
    by = dispatch_times(d)
    name, v = _pick(by, match)
    rec: dict = {"kernel": name}
    if after:
        _, marks = _pick(by, after)
        t0 = marks[-1][1]
        v = [(s, e) for s, e in v if s >= t0]
        if not v:
            raise SystemExit(f"no {match!r} dispatch after the last {after!r}")
        rec["selected"] = f"dispatches after the last {after}"
        rec["window_us_per_dispatch"] = (v[-1][1] - v[0][0]) / len(v) / 1e3
    st = _stats_us([e - s for s, e in v])
    gaps = sorted(v[i + 1][0] - v[i][1] for i in range(len(v) - 1)) or [0]
    rec.update({"dispatches": st["n"], "mean_us": st["mean"],
                "median_us": st["median"], "min_us": st["min"], "max_us": st["max"],
                "gap_median_us": gaps[len(gaps) // 2] / 1e3})
    return rec


def report_traffic(fetch: Path, write: Path, match: str, calib_match: str,
                   calib_bytes: int) -> tuple[str, dict]:
    calib_kib = calib_bytes / 1024.0
    out = {}
    lines = []
    for counter, d in (("FETCH_SIZE", fetch), ("WRITE_SIZE", write)):
        by = counter_values(d, counter)
        kname, kv = _pick(by, match)
        _, cv = _pick(by, calib_match)
        big = [v for v in cv if v >= 0.25 * calib_kib]
        if not big:
            raise SystemExit(f"no {calib_match} dispatch near {calib_kib} KiB "
                             f"in {counter}: {sorted(cv)[-5:]}")
        c_med = statistics.median(big)
        k_med = statistics.median(kv)
        factor = calib_kib / c_med
        out[counter] = {"kernel_kib_median": k_med, "kernel_dispatches": len(kv),
                        "calib_kib_median": c_med, "calib_dispatches": len(big),
                        "factor": factor, "bytes": k_med * factor * 1024.0}
        lines.append(f"{counter}: kernel {kname[:60]} median {k_med:.2f} KiB "
                     f"over {len(kv)} dispatches; calibration copy of "
                     f"{calib_kib:.0f} KiB reads {c_med:.2f} KiB "
                     f"({len(big)} dispatches) -> factor {factor:.5f} -> "
                     f"{out[counter]['bytes'] / 1e6:.4f} MB")
    total = out["FETCH_SIZE"]["bytes"] + out["WRITE_SIZE"]["bytes"]
    lines.append(f"HBM traffic per dispatch: {total:.0f} B ({total / 1e6:.4f} MB)")
    out["hbm_bytes_per_launch"] = total
    return "\n".join(lines), out


def report_counters(dirs: list[Path], matches: list[str]) -> str:
    lines = []
    for match in matches:
        lines.append(f"kernel matching {match!r}:")
        for d in dirs:
            for counter in counter_names(d):
                by = counter_values(d, counter)
                hits = [k for k in by if match in k]
                if not hits:
                    continue
                kname = max(hits, key=lambda k: len(by[k]))
                v = by[kname]
                lines.append(f"  {counter:<28} median {statistics.median(v):>14.2f}"
                             f"   ({len(v)} dispatches; {d.name})")
    return "\n".join(lines)


def _library_version() -> str | None:
    """cq_version() of the tree's built library (the build the profiled run
    loaded, when it ran from this tree); None when it cannot be loaded.
    Loading the library makes no GPU call."""
    try:
        from .. import _capi
        return _capi.version()
    except Exception:  # noqa: BLE001
        return None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir", type=Path)
    t.add_argument("--match", default=None)
    t.add_argument("--top", type=int, default=8)
    t.add_argument("--by-grid", action="store_true",
                   help="one line per (kernel, grid size)")
    t.add_argument("--shape", type=int, nargs=2, default=None)
    t.add_argument("--json-out", type=Path, default=None,
                   help="write the --match kernel's figures (and --shape) as JSON")
    t.add_argument("--after", default=None,
                   help="JSON record: only dispatches after the last one of this kernel")
    c = sub.add_parser("counters")
    c.add_argument("dirs", type=Path, nargs="+")
    c.add_argument("--match", action="append", required=True)
    f = sub.add_parser("traffic")
    f.add_argument("--fetch", type=Path, required=True)
    f.add_argument("--write", type=Path, required=True)
    f.add_argument("--match", required=True)
    f.add_argument("--calib-match", required=True)
    f.add_argument("--calib-bytes", type=int, required=True)
    f.add_argument("--shape", type=int, nargs=2, default=None)
    f.add_argument("--algorithmic-bytes", type=int, default=None)
    f.add_argument("--json-out", type=Path, default=None)
    a = ap.parse_args(argv)
    if a.cmd in ("trace", "counters"):
        lib = _library_version()
        if lib:
            print(f"library: {lib}")
    if a.cmd == "trace":
        print(report_trace(a.dir, a.match, a.top, a.by_grid))
        if a.json_out:
            if not a.match:
                raise SystemExit("--json-out needs --match")
            rec = trace_record(a.dir, a.match, a.after)
            print(json.dumps(rec, indent=1))
            rec["shape"] = list(a.shape) if a.shape else None
            rec["kernel_match"] = a.match
            rec["library"] = _library_version()
            a.json_out.write_text(json.dumps(rec, indent=1) + "\n")
        return 0
    if a.cmd == "counters":
        print(report_counters(a.dirs, a.match))
        return 0
    text, rec = report_traffic(a.fetch, a.write, a.match, a.calib_match,
                               a.calib_bytes)
    if a.algorithmic_bytes:
        rec["algorithmic_bytes"] = a.algorithmic_bytes
        rec["ratio_to_algorithmic"] = rec["hbm_bytes_per_launch"] / a.algorithmic_bytes
        text += (f"\nalgorithmic bytes {a.algorithmic_bytes} -> traffic / "
                 f"algorithmic = {rec['ratio_to_algorithmic']:.4f}")
    print(text)
    if a.json_out:
        rec["shape"] = list(a.shape) if a.shape else None
        rec["kernel_match"] = a.match
        rec["library"] = _library_version()
        a.json_out.write_text(json.dumps(rec, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
