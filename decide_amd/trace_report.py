#!/usr/bin/env python3
"""Per-kernel time per forward from a rocprofv3 kernel trace of `python3 -m decide_amd.forward --runs R`.

The traced program runs R + 1 forwards (one untimed, R timed), so each kernel's total time in the trace is divided
by R + 1; the random-init fills are left out (they run once, before the forwards), and the GEMM warm-up's single
launch of every tile variant shows as a fractional launch count. Prints a Markdown table, largest first.

Usage: python -m decide_amd.trace_report TRACE.csv --runs R [--exclude fill_normal]
"""

from __future__ import annotations

import argparse
import collections
import csv


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("trace", help="rocprofv3 *_kernel_trace.csv")
    ap.add_argument("--runs", type=int, required=True, help="timed forwards (the trace holds one more)")
    ap.add_argument("--exclude", action="append", default=["fill_normal"],
                    help="substring of kernel names to leave out (repeatable)")
    args = ap.parse_args()
    total = collections.defaultdict(float)
    count = collections.Counter()
    for row in csv.DictReader(open(args.trace)):
        name = row["Kernel_Name"]
        if any(x in name for x in args.exclude):
            continue
        total[name] += (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e6  # ms
        count[name] += 1
    per = args.runs + 1
    grand = sum(total.values()) / per
    print(f"Sum of kernel time per forward: {grand:.2f} ms.\n")
    print("| Kernel | Launches / forward | ms / forward | Share |")
    print("|---|---|---|---|")
    for name, ms in sorted(total.items(), key=lambda kv: -kv[1]):
        short = name if name.startswith("_Z") else name.split("(")[0].removeprefix("void ")
        print(f"| `{short}` | {count[name] / per:.1f} | "
              f"{ms / per:.2f} | {100 * ms / per / grand:.1f} % |")


if __name__ == "__main__":
    main()
