"""Digest of rocprofv3 CSV output into the short text summaries kept under
profiles/ (kernel durations and HBM traffic per dispatch).

    python -m fastembedr_amd.rocprof_summary trace  <kt_dir>   <command> [--last N] > profiles/<name>.txt
    python -m fastembedr_amd.rocprof_summary traffic <fetch_dir> <write_dir> <command> \
        --json profiles/<name>.json [--last N] > profiles/<name>.txt
    python -m fastembedr_amd.rocprof_summary counters <pmc_dir> <command> --names A,B [--last N]
    python -m fastembedr_amd.rocprof_summary join <kt_dir> <traffic.json> <command> --last N [--skip M]

`join` puts the kernel trace's durations beside the traffic digest's bytes
per dispatch: GB/s and the fraction of MI355X's 8 TB/s per kernel, over the
N iterations that end M iterations before the end of the trace (bench.py's
timed window is the last 20; its breakdown pass, every kernel alone, the 20
that end 750 before the end).

Counter units: FETCH_SIZE and WRITE_SIZE are read in KiB per dispatch and
scaled by what the same counter reads for a device-to-device copy of known
size in the same run (bench.py --calibrate-copy-mib).  On MI355X with
rocprofv3 (ROCm 7.x) a 512 MiB copy reads FETCH_SIZE = 262,162 KiB and
WRITE_SIZE = 524,288 KiB, i.e. factors 2.0 and 1.0.
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import re
import sys
import zlib

_OURS = re.compile(r"fehip::(?:\(anonymous namespace\)::)?(\w+)(<[^()]*>)?")


_ROCPRIM = re.compile(r"rocprim::(?:\w+::)*(\w+)")
HBM_PEAK_GBS = 8000.0


def short_name(name: str) -> str:
    m = _OURS.search(name)
    if m:
        return m.group(1) + (m.group(2) or "")
    m = _ROCPRIM.search(name)
    if m:
        # rocPRIM's kernels share a few stems (trampoline_kernel): the full
        # name's checksum tells the instantiations apart
        return f"rocprim:{m.group(1)}#{zlib.crc32(name.encode()) & 0xffffff:06x}"
    return name.split("(")[0][:60]


def ours(name: str) -> bool:
    """A kernel this library launches: its own, or a rocPRIM primitive it calls."""
    return bool(_OURS.search(name)) or "rocprim::" in name


def _one(pattern: str) -> str:
    hits = sorted(glob.glob(pattern, recursive=True))
    if not hits:
        raise FileNotFoundError(pattern)
    return hits[0]


def _stats_rows(kt_dir: str) -> list[tuple[str, int, float, float, float, float]]:
    """(name, calls, avg, min, max, total ns) per kernel, from the CSV stats
    file or, when rocprofv3 wrote its SQLite database, from its kernels view."""
    csvs = sorted(glob.glob(f"{kt_dir}/**/*kernel_stats.csv", recursive=True))
    if csvs:
        return [(r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]), float(r["MaxNs"]),
                 float(r["TotalDurationNs"])) for r in csv.DictReader(open(csvs[0]))]
    import sqlite3

    con = sqlite3.connect(_one(f"{kt_dir}/**/*.db"))
    q = ("select name, count(*), avg(end - start), min(end - start), max(end - start), sum(end - start) "
         "from kernels group by name order by sum(end - start) desc")
    return [(r[0], int(r[1]), float(r[2]), float(r[3]), float(r[4]), float(r[5])) for r in con.execute(q)]


def _window(rows: list[dict], name_key: str, last: int, skip: int = 0) -> list[dict]:
    """The dispatches (in dispatch order) of `last` iterations, the last of
    them `skip` iterations before the end: those enqueued after the update
    kernel of the iteration before them and up to the window's last update
    (one k_update per iteration), so that kernels templated on a size that
    changes during the run (the FFT lengths) are counted only in the window.
    Without enough updates, every dispatch."""
    ids = [_dispatch_order(r) for r in rows if short_name(r[name_key]).startswith("k_update")]
    if len(ids) <= last + skip:
        return rows
    first = ids[-(last + skip + 1)]
    end = ids[-(skip + 1)]
    return [r for r in rows if first < _dispatch_order(r) <= end]


def _last_rows(kt_dir: str, last: int, skip: int = 0) -> list[tuple[str, int, float, float, float, float]]:
    """As _stats_rows, over `last` iterations (_window) of the per-dispatch
    kernel trace (CSV), at most `last` dispatches per kernel."""
    per = collections.defaultdict(list)
    rows = list(csv.DictReader(open(_one(f"{kt_dir}/**/*kernel_trace.csv"))))
    rows.sort(key=_dispatch_order)
    for r in _window(rows, "Kernel_Name", last, skip):
        per[r["Kernel_Name"]].append(float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
    out = []
    for name, durs in per.items():
        d = durs[-last:]
        out.append((name, len(d), sum(d) / len(d), min(d), max(d), sum(d)))
    out.sort(key=lambda r: -r[5])
    return out


def trace(kt_dir: str, last: int = 0) -> list[str]:
    out = [f"{'kernel':34s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'total_ms':>10s}"]
    for name, calls, avg, mn, mx, tot in (_last_rows(kt_dir, last) if last > 0 else _stats_rows(kt_dir)):
        if not ours(name):
            continue
        out.append(f"{short_name(name):34s} {calls:6d} {avg / 1e3:10.2f} {mn / 1e3:10.2f} {mx / 1e3:10.2f} "
                   f"{tot / 1e6:10.2f}")
    return out


def _dispatch_order(r: dict) -> int:
    for key in ("Dispatch_Id", "Correlation_Id"):
        if r.get(key, "").strip():
            return int(r[key])
    return 0


def _counter(dir_: str, cname: str, last: int = 0):
    """Per kernel, the counter's value of each dispatch in dispatch order
    (only the last `last` iterations, _window, at most `last` dispatches per
    kernel, when last > 0), and the largest value of the calibration copy."""
    per = collections.defaultdict(list)
    calib = None
    rows = [r for r in csv.DictReader(open(_one(f"{dir_}/**/*counter_collection.csv"))) if r["Counter_Name"] == cname]
    rows.sort(key=_dispatch_order)
    for r in rows:
        v = float(r["Counter_Value"])
        if "copyBuffer" in r["Kernel_Name"] and (calib is None or v > calib):
            calib = v
    for r in _window(rows, "Kernel_Name", last) if last > 0 else rows:
        if ours(r["Kernel_Name"]):
            per[short_name(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    if last > 0:
        per = collections.defaultdict(list, {k: v[-last:] for k, v in per.items()})
    return per, calib


def counters(dir_: str, names: list[str], last: int = 0) -> list[str]:
    """Mean per dispatch of each counter, per kernel of this library."""
    cols = {c: _counter(dir_, c, last)[0] for c in names}
    kernels = sorted({k for per in cols.values() for k in per})
    out = [f"{'kernel':34s} {'dispatches':>10s} " + " ".join(f"{c:>26s}" for c in names)]
    for k in kernels:
        vals = [cols[c].get(k, []) for c in names]
        disp = max(len(v) for v in vals)
        out.append(f"{k:34s} {disp:10d} " + " ".join(f"{(sum(v) / len(v) if v else 0.0):26.1f}" for v in vals))
    return out


def traffic(fetch_dir: str, write_dir: str, copy_bytes: int, last: int = 0) -> tuple[list[str], dict]:
    fetch, fcal = _counter(fetch_dir, "FETCH_SIZE", last)
    write, wcal = _counter(write_dir, "WRITE_SIZE", last)
    if not fcal or not wcal:
        raise RuntimeError("no calibration copy found (run bench.py with --calibrate-copy-mib)")
    ffac = copy_bytes / (fcal * 1024.0)
    wfac = copy_bytes / (wcal * 1024.0)
    out = [f"calibration copy of {copy_bytes} bytes: FETCH_SIZE {fcal:.1f} KiB (factor {ffac:.3f}), "
           f"WRITE_SIZE {wcal:.1f} KiB (factor {wfac:.3f})",
           f"{'kernel':34s} {'dispatches':>10s} {'fetch_MB':>10s} {'write_MB':>10s} {'total_MB':>10s}"]
    table = {}
    for k in sorted(set(fetch) | set(write), key=lambda kk: -sum(fetch.get(kk, [0])) / max(1, len(fetch.get(kk, [0])))):
        f = fetch.get(k, [])
        w = write.get(k, [])
        fb = (sum(f) / len(f)) * 1024.0 * ffac if f else 0.0
        wb = (sum(w) / len(w)) * 1024.0 * wfac if w else 0.0
        table[k] = {"fetch_bytes": fb, "write_bytes": wb, "dispatches": len(f)}
        out.append(f"{k:34s} {len(f):10d} {fb / 1e6:10.2f} {wb / 1e6:10.2f} {(fb + wb) / 1e6:10.2f}")
    return out, {"fetch_factor": ffac, "write_factor": wfac, "kernels": table}


def join(kt_dir: str, digest: dict, last: int, skip: int = 0) -> list[str]:
    """Per kernel of the window: dispatches, mean duration, bytes per
    dispatch (digest), GB/s and the fraction of 8 TB/s; then the iteration's
    totals (time summed over the kernels, which overlap where they run beside
    each other)."""
    table = digest.get("kernels", {})
    out = [f"{'kernel':34s} {'disp':>5s} {'avg_us':>9s} {'MB/disp':>9s} {'GB/s':>8s} {'%peak':>6s} {'us/iter':>8s}"]
    tot_t = tot_b = 0.0
    for name, calls, avg, _mn, _mx, tot in _last_rows(kt_dir, last, skip):
        if not ours(name):
            continue
        k = short_name(name)
        rec = table.get(k)
        b = rec["fetch_bytes"] + rec["write_bytes"] if rec else None
        gbs = b / avg if b is not None and avg > 0 else None  # bytes per ns = GB/s
        tot_t += tot / last
        if b is not None:
            tot_b += b * calls / last
        out.append(f"{k:34s} {calls:5d} {avg / 1e3:9.2f} " + (f"{b / 1e6:9.2f} {gbs:8.0f} {100 * gbs / HBM_PEAK_GBS:6.1f}"
                                                            if b is not None else f"{'-':>9s} {'-':>8s} {'-':>6s}")
                   + f" {tot / last / 1e3:8.2f}")
    out.append(f"{'per iteration (sum)':34s} {'':5s} {'':9s} {tot_b / 1e6:9.2f} "
               f"{(tot_b / tot_t if tot_t else 0.0):8.0f} {100 * (tot_b / tot_t if tot_t else 0.0) / HBM_PEAK_GBS:6.1f}"
               f" {tot_t / 1e3:8.2f}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="what", required=True)
    t = sub.add_parser("trace")
    t.add_argument("kt_dir")
    t.add_argument("command")
    t.add_argument("--last", type=int, default=0, help="only the last N iterations' dispatches (per-dispatch trace)")
    c = sub.add_parser("traffic")
    c.add_argument("fetch_dir")
    c.add_argument("write_dir")
    c.add_argument("command")
    c.add_argument("--copy-mib", type=int, default=512)
    c.add_argument("--json", default="")
    c.add_argument("--meta", default="{}", help="JSON object stored beside the table (workload keys)")
    c.add_argument("--last", type=int, default=0, help="average only the last N iterations' dispatches")
    p = sub.add_parser("counters")
    p.add_argument("dir")
    p.add_argument("command")
    p.add_argument("--names", required=True, help="comma-separated counter names")
    p.add_argument("--last", type=int, default=0, help="average only the last N iterations' dispatches")
    j = sub.add_parser("join")
    j.add_argument("kt_dir")
    j.add_argument("digest", help="traffic digest JSON (the traffic subcommand's --json)")
    j.add_argument("command")
    j.add_argument("--last", type=int, required=True, help="iterations in the window")
    j.add_argument("--skip", type=int, default=0, help="iterations after the window's end")
    a = ap.parse_args(argv)
    if a.what == "join":
        with open(a.digest) as fh:
            dg = json.load(fh)
        lines = [f"(durations over {a.last} iterations ending {a.skip} before the trace's end; bytes per dispatch "
                 f"from {a.digest.split('/')[-1]}: {dg.get('command', '')})"] + join(a.kt_dir, dg, a.last, a.skip)
    elif a.what == "trace":
        lines = trace(a.kt_dir, a.last)
        if a.last:
            lines.insert(0, f"(durations over the last {a.last} iterations, at most {a.last} dispatches per kernel)")
    elif a.what == "counters":
        lines = counters(a.dir, a.names.split(","), a.last)
        if a.last:
            lines.insert(0, f"(mean per dispatch over the last {a.last} iterations, at most {a.last} dispatches per kernel)")
    else:
        lines, table = traffic(a.fetch_dir, a.write_dir, a.copy_mib << 20, a.last)
        if a.last:
            lines.insert(0, f"(mean per dispatch over the last {a.last} iterations, at most {a.last} dispatches per kernel)")
        if a.json:
            table.update(json.loads(a.meta))
            if a.last:
                table["window_iterations"] = a.last
            table["command"] = a.command
            with open(a.json, "w") as fh:
                json.dump(table, fh, indent=1)
    print("command: " + a.command)
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
