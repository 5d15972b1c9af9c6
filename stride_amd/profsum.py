"""Summarise rocprofv3 CSV output into the short text tables kept under profiles/.

    python -m stride_amd.profsum kernels <kernel_trace.csv> [--match k_] > summary.txt
    python -m stride_amd.profsum counters <counter_collection.csv> [--match k_]

`kernels` prints count / average / min / max duration (us) per kernel name, as
rocprofv3 --stats does; `counters` prints the average value per dispatch of each
counter per kernel (FETCH_SIZE and WRITE_SIZE are in KiB).
"""
from __future__ import annotations

import argparse
import csv
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


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["kernels", "counters"])
    ap.add_argument("csv")
    ap.add_argument("--match", default=None)
    a = ap.parse_args(argv)
    (kernels if a.mode == "kernels" else counters)(a.csv, a.match)


if __name__ == "__main__":
    main(sys.argv[1:])
