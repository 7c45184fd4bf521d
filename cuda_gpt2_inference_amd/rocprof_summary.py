"""Summaries of rocprofv3 output for the decode-attention kernels (markdown).

  python -m cuda_gpt2_inference_amd.rocprof_summary trace DIR [--title T] [--cmd C]
      per-kernel dispatch count and duration statistics from a --kernel-trace run
      (CSV output, *_kernel_trace.csv)
  python -m cuda_gpt2_inference_amd.rocprof_summary traffic FETCH_DIR WRITE_DIR [--cmd-fetch C] [--cmd-write C]
      HBM traffic per dispatch from two --pmc runs (FETCH_SIZE, then WRITE_SIZE; both in
      KiB per dispatch).  Each counter is scaled by what it reads for the calibration copy
      (__amd_rocclr_copyBuffer of a known number of bytes: the bench's PMC pass copies
      256 MiB device to device, so the copy reads and writes 256 MiB).

The traffic summary ends with one line per kernel of the form
  traffic_bytes_per_dispatch <kernel-key> <bytes>
which bench.py reads back for its roofline record.
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics
import sys
from collections import defaultdict

CALIB_BYTES = 256 << 20
CALIB_KERNEL = "__amd_rocclr_copyBuffer"


def _csv(path_glob: str):
    files = sorted(glob.glob(path_glob, recursive=True))
    if not files:
        raise SystemExit(f"no file matches {path_glob}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def short_name(name: str) -> str:
    """Kernel name without the anonymous-namespace / argument noise."""
    n = name.replace("void ", "").replace("(anonymous namespace)::", "")
    cut = n.find("((")
    if cut < 0:
        cut = n.find("(")
    return (n[:cut] if cut > 0 else n).strip()


def _key(row) -> str:
    grid = row.get("Grid_Size_X") or row.get("Grid_Size") or row.get("Grid_X") or "?"
    return f"{short_name(row['Kernel_Name'])} grid={grid}"


OWN_KERNELS = ("split_kernel", "merge_kernel", "fused_single_kernel", "cache_write", "gemv_kernel",
               "set_len_kernel")


def _phases(d: str):
    """(name, start_ns, end_ns) of the roctx ranges of a --marker-trace run, or []."""
    files = sorted(glob.glob(os.path.join(d, "**", "*marker_api_trace.csv"), recursive=True))
    res = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                name = r.get("Message") or r.get("Marker_Name") or r.get("Function") or ""
                if not name or name.startswith("roctx"):
                    continue
                res.append((name, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    return res


def _table(durs) -> list:
    out = ["| kernel (grid = work-items) | dispatches | avg µs | median µs | min µs | max µs |",
           "|---|---|---|---|---|---|"]
    for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| `{k}` | {len(v)} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
                   f"{min(v):.2f} | {max(v):.2f} |")
    return out


def trace(d: str, title: str, cmd: str, all_kernels: bool = False) -> str:
    rows = _csv(os.path.join(d, "**", "*kernel_trace.csv"))
    durs = defaultdict(list)
    spans = []
    for r in rows:
        if not all_kernels and not any(k in r["Kernel_Name"] for k in OWN_KERNELS):
            continue
        t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        durs[_key(r)].append((t1 - t0) / 1000.0)
        spans.append((t0, t1, _key(r)))
    out = [f"# {title}", "", f"Command: `{cmd}`", "", "## All dispatches", ""] + _table(durs)
    phases = _phases(d)
    if phases:
        out += ["", "## Per timed region (roctx ranges around the benchmark's timed loops)", ""]
        for name, p0, p1 in phases:
            pd = defaultdict(list)
            for t0, t1, k in spans:
                if t0 >= p0 and t1 <= p1:
                    pd[k].append((t1 - t0) / 1000.0)
            if pd:
                out += [f"### `{name}` ({(p1 - p0) / 1000.0:.1f} µs)", ""] + _table(pd) + [""]
    return "\n".join(out) + "\n"


def _counter(d: str, counter: str):
    rows = _csv(os.path.join(d, "**", "*counter_collection.csv"))
    per = defaultdict(list)
    for r in rows:
        if r.get("Counter_Name") != counter:
            continue
        per[_key(r)].append(float(r["Counter_Value"]))
    return per


def traffic(fetch_dir: str, write_dir: str, cmd_fetch: str, cmd_write: str) -> str:
    fetch_all = _counter(fetch_dir, "FETCH_SIZE")
    write_all = _counter(write_dir, "WRITE_SIZE")
    # The largest single copy dispatch is the 256 MiB calibration copy (other copies in the
    # run are smaller and may share its grid size).
    calib_f = [v for k, vs in fetch_all.items() if k.startswith(CALIB_KERNEL) for v in vs]
    calib_w = [v for k, vs in write_all.items() if k.startswith(CALIB_KERNEL) for v in vs]
    if not calib_f or not calib_w:
        raise SystemExit("calibration copy kernel not found in the counter output")
    kf = CALIB_BYTES / (max(calib_f) * 1024.0)
    kw = CALIB_BYTES / (max(calib_w) * 1024.0)
    fetch = {k: statistics.mean(v) for k, v in fetch_all.items()}
    write = {k: statistics.mean(v) for k, v in write_all.items()}
    nf = {k: len(v) for k, v in fetch_all.items()}
    out = ["# HBM traffic per dispatch (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
           f"FETCH_SIZE command: `{cmd_fetch}`", "", f"WRITE_SIZE command: `{cmd_write}`", "",
           f"Calibration: a 256 MiB device-to-device copy ({CALIB_KERNEL}) reads {max(calib_f):.0f} KiB "
           f"(FETCH_SIZE) and writes {max(calib_w):.0f} KiB (WRITE_SIZE); scale factors "
           f"fetch x{kf:.4f}, write x{kw:.4f}.", "",
           "| kernel (grid = work-items) | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes (scaled) |",
           "|---|---|---|---|---|"]
    lines = []
    for k in sorted(fetch, key=lambda x: -fetch[x]):
        if k.startswith(CALIB_KERNEL) or not any(o in k for o in OWN_KERNELS):
            continue
        f = fetch[k]
        w = write.get(k, float("nan"))
        t = f * 1024.0 * kf + w * 1024.0 * kw
        out.append(f"| `{k}` | {nf[k]} | {f:.1f} | {w:.1f} | {t:,.0f} |")
        lines.append(f"traffic_bytes_per_dispatch {k.replace(' ', '|')} {t:.0f}")
    return "\n".join(out) + "\n\n```\n" + "\n".join(lines) + "\n```\n"


def l2(d: str, cmd: str) -> str:
    """L2 (TCC) hit rate per kernel from a --pmc TCC_HIT_sum TCC_MISS_sum run."""
    hit = _counter(d, "TCC_HIT_sum")
    miss = _counter(d, "TCC_MISS_sum")
    out = ["# L2 (TCC) hit rate per dispatch (rocprofv3 TCC_HIT_sum, TCC_MISS_sum)", "",
           f"Command: `{cmd}`", "",
           "MI355X exposes no Infinity Cache (MALL) counters through rocprofv3 on this stack; the L2 figures "
           "below are the per-XCD L2 only.", "",
           "| kernel (grid = work-items) | dispatches | L2 hits | L2 misses | hit rate |", "|---|---|---|---|---|"]
    for k in sorted(hit, key=lambda x: -statistics.mean(miss.get(x, [0]))):
        if not any(o in k for o in OWN_KERNELS):
            continue
        h, m = statistics.mean(hit[k]), statistics.mean(miss.get(k, [0.0]))
        out.append(f"| `{k}` | {len(hit[k])} | {h:,.0f} | {m:,.0f} | {h / max(h + m, 1):.3f} |")
    return "\n".join(out) + "\n"


def read_traffic(md_path: str) -> dict:
    """{kernel-key: bytes} from a traffic summary written by this module."""
    res = {}
    if not os.path.exists(md_path):
        return res
    with open(md_path) as fh:
        for line in fh:
            if line.startswith("traffic_bytes_per_dispatch "):
                _, key, val = line.split()
                res[key.replace("|", " ")] = float(val)
    return res


def main(argv=None):
    p = argparse.ArgumentParser()
    sub = p.add_subparsers(dest="action", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--title", default="Kernel trace")
    t.add_argument("--cmd", default="")
    t.add_argument("--all", action="store_true", help="include kernels of other libraries")
    c = sub.add_parser("traffic")
    c.add_argument("fetch_dir")
    c.add_argument("write_dir")
    c.add_argument("--cmd-fetch", default="")
    c.add_argument("--cmd-write", default="")
    h = sub.add_parser("l2")
    h.add_argument("dir")
    h.add_argument("--cmd", default="")
    a = p.parse_args(argv)
    if a.action == "trace":
        sys.stdout.write(trace(a.dir, a.title, a.cmd, a.all))
    elif a.action == "l2":
        sys.stdout.write(l2(a.dir, a.cmd))
    else:
        sys.stdout.write(traffic(a.fetch_dir, a.write_dir, a.cmd_fetch, a.cmd_write))


if __name__ == "__main__":
    main()
