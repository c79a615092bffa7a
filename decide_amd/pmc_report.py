#!/usr/bin/env python3
"""Per-shape hardware counters of the prefill GEMM path, from rocprofv3 --pmc runs of the shape report.

Three passes of `python -m decide_amd.shape_report --markers` under rocprofv3 (a counter set per pass,
as the hardware allows):

    rocprofv3 --pmc MfmaUtil MfmaFlopsF16 -d D/mfma -o mfma --output-format csv -- python3 -m decide_amd.shape_report --iters 40 --markers
    rocprofv3 --pmc FETCH_SIZE -d D/fetch -o fetch --output-format csv -- python3 -m decide_amd.shape_report --iters 40 --markers
    rocprofv3 --pmc WRITE_SIZE -d D/write -o write --output-format csv -- python3 -m decide_amd.shape_report --iters 40 --markers
    python3 -m decide_amd.pmc_report --dir D --md D/pmc_shapes.md

The shape report puts a memset (`__amd_rocclr_fillBufferAligned`) before each shape; the dispatches
between marker i and marker i + 1 are shape i's launches (its GEMM kernels, and the split-K reduce where
the plan has one). Per shape, over all its launches:

* MFMA utilisation: AMD's `MfmaUtil` (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE × SIMDs), weighted by
  dispatch duration;
* MFMA TFLOP/s from the counted fp16 MFMA operations (`MfmaFlopsF16`) over the kernels' time, and those
  counted flops over the algorithmic 2·M·N·K (above 1: padding rows and columns the tiles compute);
* HBM bytes: FETCH_SIZE and WRITE_SIZE in KiB scaled by what they read for the calibration copy of
  known size (FETCH_SIZE counts 64 B per 128 B line read on gfx950), over the kernels' time, against
  MI355X's 8 TB/s.

Time here is the sum of the kernels' own durations (End − Start) under the counter runs, which serialise
dispatches: it excludes launch gaps and runs at the clock a lone kernel holds.
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import os
import sys

if __package__ in (None, ""):
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from decide_amd.shape_report import CALIBRATION_BYTES, PEAK_GBS, PEAK_TFLOPS, SHAPES, algorithmic  # noqa: E402

MARKER = "__amd_rocclr_fillBufferAligned"
COPY = "__amd_rocclr_copyBuffer"
SETUP = "dh::fill_normal_f16_kernel"  # the report's own random fills (the head's table), not measured


def read_pass(path_glob: str):
    """Dispatches in order: [(name, start, end, {counter: value})]."""
    files = glob.glob(path_glob)
    if not files:
        raise SystemExit(f"no counter file matches {path_glob}")
    by_id = collections.OrderedDict()
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                key = (r["Agent_Id"], r["Dispatch_Id"])
                d = by_id.setdefault(key, [r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]), {}])
                d[3][r["Counter_Name"]] = d[3].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return sorted(by_id.values(), key=lambda d: d[1])


def segments(dispatches):
    """The calibration copy's counters, then the dispatches after each marker memset up to the next one
    (memsets before the calibration copy belong to the report's own set-up)."""
    segs, cur, calib = [], None, None
    for name, t0, t1, c in dispatches:
        if calib is None:
            if name.startswith(COPY):
                calib = c
        elif name.startswith(MARKER):
            cur = []
            segs.append(cur)
        elif cur is not None and not name.startswith(SETUP) and not name.startswith(COPY):
            cur.append((name, t0, t1, c))  # (copies after the calibration are the head's input uploads)
    return segs, calib


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--dir", required=True, help="directory holding the mfma/, fetch/ and write/ pass outputs")
    ap.add_argument("--md", default="")
    args = ap.parse_args()
    mf, cal_m = segments(read_pass(os.path.join(args.dir, "mfma", "*counter_collection.csv")))
    fe, cal_f = segments(read_pass(os.path.join(args.dir, "fetch", "*counter_collection.csv")))
    wr, cal_w = segments(read_pass(os.path.join(args.dir, "write", "*counter_collection.csv")))
    names = [s[0] for s in SHAPES] + ["C4 head 24x64 (bf16 gather)"]
    if not (len(mf) == len(fe) == len(wr) == len(names)):
        raise SystemExit(f"marker count mismatch: {len(mf)} {len(fe)} {len(wr)} for {len(names)} shapes")
    fscale = CALIBRATION_BYTES / (cal_f["FETCH_SIZE"] * 1024)
    wscale = CALIBRATION_BYTES / (cal_w["WRITE_SIZE"] * 1024)
    lines = [f"Byte scale from the {CALIBRATION_BYTES:,}-byte calibration copy: fetch × {fscale:.4f}, "
             f"write × {wscale:.4f}.", "",
             "| Shape | Launches | µs per launch | MfmaUtil % | MFMA TFLOP/s (counted) | % MFMA peak | "
             "counted ÷ algorithmic flops | HBM GB/s | % HBM peak |",
             "|---|---|---|---|---|---|---|---|---|"]
    shape_args = {s[0]: s for s in SHAPES}
    for i, name in enumerate(names):
        segm, segf, segw = mf[i], fe[i], wr[i]
        tm = sum(t1 - t0 for _, t0, t1, _ in segm) * 1e-9
        util = sum(c.get("MfmaUtil", 0.0) * (t1 - t0) for _, t0, t1, c in segm) * 1e-9 / tm
        flops = sum(c.get("MfmaFlopsF16", 0.0) for *_, c in segm)
        tf_ = sum(t1 - t0 for _, t0, t1, _ in segf) * 1e-9
        tw_ = sum(t1 - t0 for _, t0, t1, _ in segw) * 1e-9
        fetch = sum(c.get("FETCH_SIZE", 0.0) for *_, c in segf) * 1024 * fscale
        write = sum(c.get("WRITE_SIZE", 0.0) for *_, c in segw) * 1024 * wscale
        # launches: count the dispatches of the shape's first kernel name
        first = segm[0][0] if segm else ""
        launches = sum(1 for d in segm if d[0] == first)
        hbm = fetch / tf_ + write / tw_  # bytes per second, each pass over its own kernel time
        if name in shape_args:
            _, m, k, members = shape_args[name]
            alg, _ = algorithmic(m, k, members)
            ratio = f"{flops / (alg * launches):.3f}"
        else:
            ratio = "—"
        lines.append(f"| {name} | {launches} | {tm / launches * 1e6:.1f} | {util:.1f} | {flops / tm / 1e12:.0f} | "
                     f"{100 * flops / tm / 1e12 / PEAK_TFLOPS:.1f} | {ratio} | "
                     f"{hbm / 1e9:.0f} | {100 * hbm / 1e9 / PEAK_GBS:.1f} |")
    table = "\n".join(lines)
    print(table)
    if args.md:
        with open(args.md, "w") as f:
            f.write(table + "\n")


if __name__ == "__main__":
    main()
