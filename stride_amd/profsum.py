"""Summarise rocprofv3 CSV output into the short text tables kept under profiles/.

    python -m stride_amd.profsum kernels <kernel_trace.csv> [--match k_] > summary.txt
    python -m stride_amd.profsum counters <counter_collection.csv> [--match k_]
    python -m stride_amd.profsum traffic <fetch counter_collection.csv> --write-csv <write csv> \
        --calib-match neg --calib-bytes 536870912 > traffic.json

`kernels` prints count / average / min / max duration (us) per kernel name, as
rocprofv3 --stats does; `counters` prints the average value per dispatch of each
counter per kernel (FETCH_SIZE and WRITE_SIZE are in KiB). `traffic` turns a
FETCH_SIZE run and a WRITE_SIZE run into HBM bytes per dispatch, each counter
scaled by what it reads for a calibration kernel that moves a known number of
bytes each way (a plain copy), and prints the JSON that bench.py reads.
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict


def short(name: str) -> str:
    name = name.replace("stride_tc::", "")
    name = re.sub(r"\(stride_tc::Geometry.*$|\(Geometry.*$", "", name)
    name = re.sub(r"^void ", "", name)
    return name[:140]


def kernels(path: str, match: str | None) -> None:
    rows = defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            n = short(r["Kernel_Name"])
            if match and match not in n:
                continue
            rows[n].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print(f"{'kernel':<90} {'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'total_us':>12}")
    for n, d in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        print(f"{n:<90} {len(d):>6} {sum(d) / len(d):>10.2f} {min(d):>10.2f} {max(d):>10.2f} {sum(d):>12.1f}")


def counters(path: str, match: str | None) -> None:
    vals = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(lambda: defaultdict(set))
    with open(path) as f:
        for r in csv.DictReader(f):
            n = short(r["Kernel_Name"])
            if match and match not in n:
                continue
            c = r["Counter_Name"]
            vals[n][c] += float(r["Counter_Value"])
            disp[n][c].add(r["Dispatch_Id"])
    print(f"{'kernel':<90} {'counter':>12} {'dispatches':>10} {'avg_per_dispatch':>18}")
    for n in sorted(vals):
        for c in sorted(vals[n]):
            k = len(disp[n][c])
            print(f"{n:<90} {c:>12} {k:>10} {vals[n][c] / k:>18.1f}")


def per_dispatch(path: str, counter: str) -> dict:
    """Average value of `counter` per dispatch, by short kernel name."""
    vals = defaultdict(float)
    disp = defaultdict(set)
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            n = short(r["Kernel_Name"])
            vals[n] += float(r["Counter_Value"])
            disp[n].add(r["Dispatch_Id"])
    return {n: vals[n] / len(disp[n]) for n in vals}


def traffic(fetch_csv: str, write_csv: str, calib_match: str, calib_bytes: int, match: str | None) -> None:
    fetch = per_dispatch(fetch_csv, "FETCH_SIZE")
    write = per_dispatch(write_csv, "WRITE_SIZE")
    cal = [n for n in fetch if calib_match in n]
    if len(cal) != 1 or cal[0] not in write:
        raise SystemExit(f"need exactly one calibration kernel matching {calib_match!r} in both runs, found {cal}")
    fs = calib_bytes / (fetch[cal[0]] * 1024.0)
    ws = calib_bytes / (write[cal[0]] * 1024.0)
    out = {
        "source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE --kernel-trace, one run each",
        "calibration": {"kernel": cal[0], "bytes_each_way": calib_bytes, "fetch_scale": round(fs, 4),
                        "write_scale": round(ws, 4)},
        "kernels": {},
    }
    for n in sorted(fetch):
        if n == cal[0] or (match and match not in n) or n not in write:
            continue
        fb, wb = fetch[n] * 1024.0 * fs, write[n] * 1024.0 * ws
        out["kernels"][n] = {"fetch_bytes": int(fb), "write_bytes": int(wb), "hbm_bytes": int(fb + wb)}
    print(json.dumps(out, indent=1))


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["kernels", "counters", "traffic"])
    ap.add_argument("csv")
    ap.add_argument("--match", default=None)
    ap.add_argument("--write-csv", default=None)
    ap.add_argument("--calib-match", default="neg")
    ap.add_argument("--calib-bytes", type=int, default=512 << 20)
    a = ap.parse_args(argv)
    if a.mode == "traffic":
        traffic(a.csv, a.write_csv, a.calib_match, a.calib_bytes, a.match)
    else:
        (kernels if a.mode == "kernels" else counters)(a.csv, a.match)


if __name__ == "__main__":
    main(sys.argv[1:])
