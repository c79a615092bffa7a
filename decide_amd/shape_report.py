#!/usr/bin/env python3
"""Per-shape throughput of the prefill GEMM path on this GPU, against MI355X peaks.

For every GEMM shape of the benchmark configurations (C1 single GEMM, C2 MLP
block, C3 grouped projections, C4 M = 2,307 layer + candidate head, and the
pruned last layer's answer-row GEMMs) this times back-to-back launches with
HIP events, weights rotated through enough copies (> 256 MB) that they stream
from HBM and not the Infinity Cache, and reports per launch:

* time (mean of the launches, and the median of 8 sub-batches),
* algorithmic TFLOP/s (2·M·N·K) and its fraction of dense fp16 MFMA peak,
* algorithmic GB/s (2·M·K + 2·N·K + output bytes [+ 4·M·N read for AddF32];
  a grouped launch counts X once) and its fraction of HBM peak,
* which roofline binds (arithmetic intensity against the 315 flop/B ridge).

decide reports its GEMMs the same way per shape in its planner notes
(crates/decide-metal/src/gemm_configs.rs:247-309); the algorithmic byte/flop
formulas follow its GEMM contract (kernels/gemm.rs:126-137).

With --markers (for runs under rocprofv3 --pmc), one device-to-device copy of
CALIBRATION_BYTES comes first (the reference for the FETCH_SIZE / WRITE_SIZE
byte scale), and a 1 MB memset runs before each shape, so that
decide_amd/pmc_report.py can cut the counter dispatch stream into shapes.

Usage: python -m decide_amd.shape_report [--iters 200] [--json out.json] [--md out.md] [--markers]
"""

from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

if __package__ in (None, ""):
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from decide_amd import hip, synth  # noqa: E402
from decide_amd.hip import DeviceArray, Event, Stream  # noqa: E402
from decide_amd.kernels import Epilogue, Kernels, fill_normal_f16  # noqa: E402

PEAK_TFLOPS = 2516.6
PEAK_GBS = 8000.0
RIDGE = PEAK_TFLOPS * 1e12 / (PEAK_GBS * 1e9)
POOL_BYTES = 640 << 20
MIN_ROTATION_BYTES = 300 << 20
CALIBRATION_BYTES = 94371840  # one device-to-device copy under --markers (the counter byte-scale reference)
MARKER_BYTES = 1 << 20  # memset between shapes under --markers

# (name, M, K, [(N, epi), ...]) — one entry = one launch (a grouped launch if several members)
SHAPES = [
    ("C1 proj StoreF32", 276, 2560, [(9216, Epilogue.StoreF32)]),
    ("C1 proj StoreF16", 276, 2560, [(9216, Epilogue.StoreF16)]),
    ("C2 gate|up SwiGLU", 603, 2560, [(18432, Epilogue.SwigluF16)]),
    ("C2 down +residual", 603, 9216, [(2560, Epilogue.AddF32)]),
    ("C3 attn Q|K|V grouped", 603, 2560, [(4096, Epilogue.StoreF32), (1024, Epilogue.StoreF32),
                                          (1024, Epilogue.StoreF32)]),
    ("C3 attn q|gate|k|v", 603, 2560, [(10240, Epilogue.StoreF32)]),
    ("C3 GDN qkv|z|b|a", 603, 2560, [(12352, Epilogue.StoreF32)]),
    ("C3 out-proj +residual", 603, 4096, [(2560, Epilogue.AddF32)]),
    ("C4 gate|up SwiGLU", 2307, 2560, [(18432, Epilogue.SwigluF16)]),
    ("C4 down +residual", 2307, 9216, [(2560, Epilogue.AddF32)]),
    ("C4 attn Q|K|V grouped", 2307, 2560, [(4096, Epilogue.StoreF32), (1024, Epilogue.StoreF32),
                                           (1024, Epilogue.StoreF32)]),
    ("C4 attn q|gate|k|v", 2307, 2560, [(10240, Epilogue.StoreF32)]),
    ("C4 GDN qkv|z|b|a", 2307, 2560, [(12352, Epilogue.StoreF32)]),
    ("C4 out-proj +residual", 2307, 4096, [(2560, Epilogue.AddF32)]),
    ("pruned q|gate (3 rows)", 3, 2560, [(8192, Epilogue.StoreF32)]),
    ("pruned k|v (3 rows)", 3, 2560, [(2048, Epilogue.StoreF32)]),
    ("pruned o (3 rows)", 3, 4096, [(2560, Epilogue.AddF32)]),
    ("pruned gate|up (3 rows)", 3, 2560, [(18432, Epilogue.SwigluF16)]),
    ("pruned down (3 rows)", 3, 9216, [(2560, Epilogue.AddF32)]),
    ("answer rows gate|up (16)", 16, 2560, [(18432, Epilogue.SwigluF16)]),
]


def out_elem_bytes(epi: Epilogue) -> float:
    return {Epilogue.StoreF32: 4, Epilogue.StoreF16: 2, Epilogue.AddF32: 8, Epilogue.SwigluF16: 1}[epi]


def algorithmic(m: int, k: int, members) -> tuple[float, float]:
    """flops and bytes of one launch (SwiGLU writes N/2 fp16 = 1 byte per accumulator column)."""
    fl = sum(2.0 * m * n * k for n, _ in members)
    by = 2.0 * m * k + sum(2.0 * n * k + out_elem_bytes(e) * m * n for n, e in members)
    return fl, by


def head_shape(k: Kernels, st: Stream, iters: int):
    """C4's candidate head: 24 answer rows × 64 candidate ids over a 151,936-row bf16 table."""
    rows, cands, hidden, vocab = 24, 64, 2560, 151936
    s = st.handle
    table = DeviceArray((vocab, hidden), np.uint16)
    fill_normal_f16(k.ctx, s, (table, 0), vocab * hidden, 31, 0.02)  # any 16-bit pattern will do
    x = DeviceArray.from_numpy(synth.normal_f32(synth.seed_for(32), (rows, hidden), 1.0))
    w = DeviceArray.from_numpy(synth.normal_f32(synth.seed_for(33), (hidden,), 0.02))
    ids = synth.uniform_ids(synth.seed_for(34), rows * cands, vocab).astype(np.uint32)
    cand = DeviceArray.from_numpy(ids)
    ncand = DeviceArray.from_numpy(np.full(rows, cands, np.uint32))
    logits = DeviceArray((rows * cands,), np.float32)
    run = lambda: k.head.final_head(s, (x, 0), (w, 0), (table, 0), (cand, 0), (ncand, 0), (logits, 0), rows,
                                    hidden, cands)
    us = time_launches(run, st, iters)
    fl = 2.0 * rows * cands * hidden
    by = 4.0 * rows * hidden + 2.0 * rows * cands * hidden + 4.0 * rows * cands + 4.0 * rows * cands
    table.free()
    return us, fl, by


def time_launches(run, st: Stream, iters: int):
    for _ in range(3):
        run()
    st.synchronize()
    batches = 8
    per = max(1, iters // batches)
    times = []
    for _ in range(batches):
        e0, e1 = Event(), Event()
        e0.record(st.handle)
        for _ in range(per):
            run()
        e1.record(st.handle)
        e1.synchronize()
        times.append(e0.elapsed_ms(e1) * 1e3 / per)
        e0.destroy()
        e1.destroy()
    return float(np.mean(times)), float(np.median(times))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--json", default="")
    ap.add_argument("--md", default="")
    ap.add_argument("--markers", action="store_true", help="calibration copy + a memset before each shape")
    args = ap.parse_args()
    if not hip.available():
        sys.exit("no GPU")
    k = Kernels()
    st = Stream()
    s = st.handle
    pool = DeviceArray((POOL_BYTES // 2,), np.float16)
    fill_normal_f16(k.ctx, s, (pool, 0), POOL_BYTES // 2, 7, 0.02)
    maxm, maxk = 2307, 9216
    maxn = max(sum(n for n, _ in mem) for _, _, _, mem in SHAPES)
    x = DeviceArray((maxm * maxk,), np.float16)
    fill_normal_f16(k.ctx, s, (x, 0), maxm * maxk, 8, 1.0)
    y = DeviceArray((maxm * maxn,), np.float32)
    y.zero_()
    k.gemm.warm_up(s, maxm)
    st.synchronize()
    marker_buf = None
    if args.markers:
        src = DeviceArray((CALIBRATION_BYTES // 2,), np.float16)
        dst = DeviceArray((CALIBRATION_BYTES // 2,), np.float16)
        src.zero_()
        dst.copy_(src)
        hip.synchronize()
        src.free()
        dst.free()
        marker_buf = DeviceArray((MARKER_BYTES // 4,), np.float32)

    def marker():
        if marker_buf is not None:
            marker_buf.zero_()
            hip.synchronize()

    loaded = k.gemm.fast_pipelines()
    results = []
    for name, m, kk, members in SHAPES:
        marker()
        wbytes = sum(n * kk * 2 for n, _ in members)
        copies = max(1, min(POOL_BYTES // wbytes, -(-MIN_ROTATION_BYTES // wbytes)))
        state = {"i": 0}
        if len(members) == 1:
            n, epi = members[0]
            ldy = n // 2 if epi == Epilogue.SwigluF16 else n

            def run(n=n, epi=epi, ldy=ldy):
                c = state["i"] % copies
                state["i"] += 1
                k.gemm.gemm(s, (x, 0), (pool, c * wbytes), (y, 0), m, n, kk, kk, kk, ldy, epi)
        else:
            def run():
                c = state["i"] % copies
                state["i"] += 1
                woff, yoff, mem = c * wbytes, 0, []
                for n, epi in members:
                    mem.append(((pool, woff), kk, n, (y, yoff), n, epi))
                    woff += n * kk * 2
                    yoff += m * n * 4
                k.gemm.gemm_grouped(s, (x, 0), kk, m, kk, mem)
        mean_us, med_us = time_launches(run, st, args.iters)
        fl, by = algorithmic(m, kk, members)
        plan = k.gemm.plan(m, sum(n for n, _ in members), kk, members[0][1]) if len(members) == 1 else None
        results.append(dict(name=name, m=m, k=kk, n=[n for n, _ in members], epi=[e.name for _, e in members],
                            us_mean=mean_us, us_median=med_us, flops=fl, bytes=by, rotation=copies, plan=plan))
    assert k.gemm.fast_pipelines() == loaded, "a GEMM kernel was loaded after warm-up"
    marker()
    us, fl, by = head_shape(k, st, args.iters)
    results.append(dict(name="C4 head 24x64 (bf16 gather)", m=24, k=2560, n=[64], epi=["head"], us_mean=us[0],
                        us_median=us[1], flops=fl, bytes=by, rotation=1, plan=None))
    lines = ["| Shape | M | K | N | µs (median) | TFLOP/s | % MFMA peak | GB/s | % HBM peak | Bound |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    for r in results:
        t = r["us_median"] * 1e-6
        tf, gbs = r["flops"] / t / 1e12, r["bytes"] / t / 1e9
        bound = "mfma" if r["flops"] / r["bytes"] > RIDGE else "hbm"
        r.update(tflops=tf, pct_mfma=100 * tf / PEAK_TFLOPS, gbs=gbs, pct_hbm=100 * gbs / PEAK_GBS, bound=bound)
        lines.append(f"| {r['name']} | {r['m']} | {r['k']} | {'+'.join(map(str, r['n']))} | {r['us_median']:.1f} | "
                     f"{tf:.0f} | {r['pct_mfma']:.1f} | {gbs:.0f} | {r['pct_hbm']:.1f} | {bound} |")
        print(json.dumps({kk: (round(v, 3) if isinstance(v, float) else v) for kk, v in r.items()}), flush=True)
    table = "\n".join(lines)
    print(table, flush=True)
    if args.json:
        os.makedirs(os.path.dirname(args.json) or ".", exist_ok=True)
        with open(args.json, "w") as f:
            json.dump(results, f, indent=1)
    if args.md:
        os.makedirs(os.path.dirname(args.md) or ".", exist_ok=True)
        with open(args.md, "w") as f:
            f.write(table + "\n")


if __name__ == "__main__":
    main()
