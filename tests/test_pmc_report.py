"""Host logic of decide_amd/pmc_report.py: the dispatch stream is cut into shapes at the marker memsets
after the calibration copy, set-up fills and uploads are skipped, and counters sum per shape."""

import csv
import os

from decide_amd import pmc_report


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Agent_Id", "Dispatch_Id", "Kernel_Name", "Start_Timestamp",
                                          "End_Timestamp", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def _stream(counter, per_kernel):
    """set-up memset, calibration copy, then 2 shapes: marker, 2 launches of a GEMM (+ a set-up fill)."""
    seq = [("__amd_rocclr_fillBufferAligned", 0.0), ("__amd_rocclr_copyBuffer", 1000.0),
           ("__amd_rocclr_fillBufferAligned", 0.0), ("gemm_a", per_kernel), ("gemm_a", per_kernel),
           ("__amd_rocclr_fillBufferAligned", 0.0), ("dh::fill_normal_f16_kernel(x)", 99.0),
           ("__amd_rocclr_copyBuffer", 7.0), ("gemm_b", 2 * per_kernel), ("gemm_b", 2 * per_kernel)]
    rows, t = [], 0
    for i, (name, v) in enumerate(seq):
        rows.append(dict(Agent_Id=1, Dispatch_Id=i, Kernel_Name=name, Start_Timestamp=t, End_Timestamp=t + 100,
                         Counter_Name=counter, Counter_Value=v))
        t += 1000
    return rows


def test_segments_skip_setup_and_sum_per_shape(tmp_path):
    path = os.path.join(tmp_path, "x_counter_collection.csv")
    _write(path, _stream("FETCH_SIZE", 5.0))
    segs, calib = pmc_report.segments(pmc_report.read_pass(path))
    assert calib == {"FETCH_SIZE": 1000.0}
    assert [[d[0] for d in s] for s in segs] == [["gemm_a", "gemm_a"], ["gemm_b", "gemm_b"]]
    assert sum(d[3]["FETCH_SIZE"] for d in segs[1]) == 20.0
    assert sum(d[2] - d[1] for d in segs[0]) == 200
