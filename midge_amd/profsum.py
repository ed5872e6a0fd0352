"""Summaries of rocprofv3 CSV output for profiles/ (kernel times and HBM
traffic), so the figures quoted by bench.py can be traced to a profiler run.

    python -m midge_amd.profsum stats  <kernel_stats.csv> [--top N]
    python -m midge_amd.profsum traffic <fetch counter_collection.csv> <write counter_collection.csv>
                                        --kernel REGEX --copy-bytes N [--json OUT]

    python -m midge_amd.profsum counters <counter_collection.csv> --kernel REGEX

`counters` averages every counter of the file per dispatch over the
dispatches whose kernel name matches REGEX (one line per kernel name).

`traffic` averages FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over the
dispatches whose kernel name matches REGEX, and scales each by the ratio the
same counter shows for the runtime's device-to-device copy kernel of N bytes
(which reads N and writes N bytes), giving HBM bytes per launch.
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict


def _rows(path: str) -> list[dict]:
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _col(row: dict, *names: str) -> str:
    for n in names:
        if n in row:
            return row[n]
    raise KeyError(f"none of {names} in {list(row)}")


def stats(path: str, top: int) -> str:
    rows = _rows(path)
    out = ["| kernel | calls | avg (us) | min (us) | max (us) | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in rows[:top]:
        name = _col(r, "Name", "KERNEL_NAME", "Kernel_Name")
        out.append("| {} | {} | {:.2f} | {:.2f} | {:.2f} | {:.1f} |".format(
            name.replace("|", "\\|")[:90], _col(r, "Calls", "CALLS"),
            float(_col(r, "AverageNs", "AVERAGE_NS")) / 1e3, float(_col(r, "MinNs", "MIN_NS")) / 1e3,
            float(_col(r, "MaxNs", "MAX_NS")) / 1e3, float(_col(r, "Percentage", "PERCENTAGE"))))
    return "\n".join(out)


def _per_kernel(path: str, counter: str) -> dict[str, list[float]]:
    acc: dict[str, list[float]] = defaultdict(list)
    for r in _rows(path):
        if _col(r, "Counter_Name", "COUNTER_NAME") != counter:
            continue
        acc[_col(r, "Kernel_Name", "KERNEL_NAME")].append(float(_col(r, "Counter_Value", "COUNTER_VALUE")))
    return acc


def traffic(fetch_csv: str, write_csv: str, kernel: str, copy_bytes: int) -> dict:
    res = {"kernel_regex": kernel, "copy_bytes": copy_bytes}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        per = _per_kernel(path, counter)
        copy = [v for k, vs in per.items() if "copyBuffer" in k for v in vs]
        big = [v for v in copy if v * 1024 > copy_bytes / 2]   # the calibration copies, not small uploads
        if not big:
            raise SystemExit(f"{counter}: no copy dispatch of ~{copy_bytes} B found in {path}")
        kib_copy = sum(big) / len(big)
        factor = copy_bytes / (kib_copy * 1024.0)
        hits = [v for k, vs in per.items() if re.search(kernel, k) for v in vs]
        if not hits:
            raise SystemExit(f"{counter}: no dispatch of /{kernel}/ in {path}")
        kib = sum(hits) / len(hits)
        res[counter] = {"kib_per_dispatch": kib, "dispatches": len(hits), "copy_kib": kib_copy,
                        "copy_dispatches": len(big), "scale": factor, "bytes_per_dispatch": kib * 1024.0 * factor}
    res["traffic_bytes"] = res["FETCH_SIZE"]["bytes_per_dispatch"] + res["WRITE_SIZE"]["bytes_per_dispatch"]
    return res


def counters(path: str, kernel: str) -> str:
    acc: dict[tuple[str, str], list[float]] = defaultdict(list)
    for r in _rows(path):
        k = _col(r, "Kernel_Name", "KERNEL_NAME")
        if re.search(kernel, k):
            acc[(k, _col(r, "Counter_Name", "COUNTER_NAME"))].append(float(_col(r, "Counter_Value", "COUNTER_VALUE")))
    if not acc:
        raise SystemExit(f"no dispatch of /{kernel}/ in {path}")
    out = ["| kernel | counter | dispatches | mean per dispatch |", "|---|---|---|---|"]
    for (k, c), vs in sorted(acc.items()):
        out.append(f"| {k.replace('|', chr(92) + '|')[:70]} | {c} | {len(vs)} | {sum(vs) / len(vs):.6g} |")
    return "\n".join(out)


def main() -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("csv")
    a.add_argument("--top", type=int, default=15)
    b = sub.add_parser("traffic")
    b.add_argument("fetch_csv")
    b.add_argument("write_csv")
    b.add_argument("--kernel", required=True)
    b.add_argument("--copy-bytes", type=int, required=True)
    b.add_argument("--json")
    c = sub.add_parser("counters")
    c.add_argument("csv")
    c.add_argument("--kernel", required=True)
    args = ap.parse_args()
    if args.cmd == "stats":
        print(stats(args.csv, args.top))
    elif args.cmd == "counters":
        print(counters(args.csv, args.kernel))
    else:
        r = traffic(args.fetch_csv, args.write_csv, args.kernel, args.copy_bytes)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(r, f, indent=1)
        print(json.dumps(r, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
