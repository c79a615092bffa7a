#!/usr/bin/env python3
"""Measure every (tile variant, split-K) of the GEMM planner on this GPU for decide's engine shapes.

The MI355X counterpart of decide's tuning workflow for its M1 Pro table
(crates/decide-metal/src/gemm_configs.rs:247-309): time each compiled variant
and split factor with HIP events over back-to-back launches, weights rotated
through enough copies (> 256 MB) that they stream from HBM rather than the
Infinity Cache, and print the fastest choice per (K, N, M) as the C++ rows of
the planner's measured table (decide_amd/csrc/plan.cpp) plus a JSON record.

Usage: python -m decide_amd.tune_gemm [--out results.json] [--ms 1,8,603] [--shapes K:N,...]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

if __package__ in (None, ""):
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from decide_amd import hip  # noqa: E402
from decide_amd.hip import DeviceArray, Event, Stream  # noqa: E402
from decide_amd.kernels import Epilogue, Kernels, fill_normal_f16, variants  # noqa: E402

# decide's engine GEMM shapes (K, N) (gemm_configs.rs:385) plus BASELINE's Q/K/V group and
# the un-interleaved MLP half, with the epilogue each runs under in the forward.
ENGINE_SHAPES = [
    (2560, 12352, Epilogue.StoreF32),  # GDN in-projection qkv|z|b|a
    (2560, 10240, Epilogue.StoreF32),  # attention in-projection q|gate|k|v
    (2560, 18432, Epilogue.SwigluF16),  # MLP gate|up
    (4096, 2560, Epilogue.AddF32),  # attention / GDN out-projection
    (9216, 2560, Epilogue.AddF32),  # MLP down
    (2560, 2048, Epilogue.StoreF32),  # pruned layer k|v
    (2560, 8192, Epilogue.StoreF32),  # pruned layer q|gate
    (2560, 6144, Epilogue.StoreF32),  # BASELINE attention group Q|K|V
    (2560, 9216, Epilogue.StoreF32),
]
DEFAULT_MS = [1, 3, 8, 16, 24, 48, 96, 163, 276, 490, 603, 1024, 2307]
SPLITS = [1, 2, 3, 4, 6, 8]
POOL_BYTES = 640 << 20


TIE = 0.02  # choices this close to the fastest count as ties


def padded_area(vi: dict, m: int, n: int) -> int:
    """Output area the tiles of a variant cover, padding rows and columns included."""
    return -(-m // vi["bm"]) * vi["bm"] * -(-n // vi["bn"]) * vi["bn"]


def pick(rows, m: int, n: int):
    """The fastest (time, variant, splits), except that among choices within TIE of it the one
    with the least padded tile area wins: in sustained runs the chip is power-limited, and MFMA work
    on padding rows costs energy that a burst timing does not show."""
    vs = variants()
    close = [r for r in rows if r[0] <= rows[0][0] * (1 + TIE)]
    return min(close, key=lambda r: (padded_area(vs[r[1]], m, n), r[0]))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", default="gpurun_out/tune_gemm.json")
    ap.add_argument("--ms", default=",".join(map(str, DEFAULT_MS)))
    ap.add_argument("--shapes", default="", help="K:N pairs (default: the engine shapes)")
    ap.add_argument("--iters", type=int, default=12)
    args = ap.parse_args()
    if not hip.available():
        sys.exit("no GPU")
    ms = [int(v) for v in args.ms.split(",") if v]
    shapes = ENGINE_SHAPES
    if args.shapes:
        want = {tuple(int(x) for x in kv.split(":")) for kv in args.shapes.split(",")}
        shapes = [s for s in ENGINE_SHAPES if (s[0], s[1]) in want]
    k = Kernels()
    st = Stream()
    s = st.handle
    pool = DeviceArray((POOL_BYTES // 2,), np.float16)
    fill_normal_f16(k.ctx, s, (pool, 0), POOL_BYTES // 2, 7, 0.02)
    maxm, maxk, maxn = max(ms), max(sh[0] for sh in shapes), max(sh[1] for sh in shapes)
    x = DeviceArray((maxm * maxk,), np.float16)
    fill_normal_f16(k.ctx, s, (x, 0), maxm * maxk, 8, 1.0)
    y = DeviceArray((maxm * maxn,), np.float32)
    y.zero_()
    k.gemm.warm_up(s, maxm)
    st.synchronize()
    nvar = len(variants())
    # Let the clocks settle first: the first ~300 launches of sustained MFMA load run ~10 % slower.
    kk0, n0, epi0 = shapes[0]
    for i in range(400):
        k.gemm.gemm(s, (x, 0), (pool, 0), (y, 0), max(ms), n0, kk0, kk0, kk0, n0 // 2 if epi0 == Epilogue.SwigluF16 else n0,
                    epi0)
    st.synchronize()
    results = []
    t_start = time.time()
    for (kk, n, epi) in shapes:
        wbytes = n * kk * 2
        copies = max(1, min(POOL_BYTES // wbytes, (400 << 20) // wbytes + 1))
        ldy = n // 2 if epi == Epilogue.SwigluF16 else n
        for m in ms:
            def timeit():
                for i in range(3):
                    k.gemm.gemm(s, (x, 0), (pool, (i % copies) * wbytes), (y, 0), m, n, kk, kk, kk, ldy, epi)
                e0, e1 = Event(), Event()
                e0.record(s)
                for i in range(args.iters):
                    k.gemm.gemm(s, (x, 0), (pool, (i % copies) * wbytes), (y, 0), m, n, kk, kk, kk, ldy, epi)
                e1.record(s)
                e1.synchronize()
                t = e0.elapsed_ms(e1) / args.iters * 1e3
                e0.destroy()
                e1.destroy()
                return t
            rows = []
            for v in range(nvar):
                vi = variants()[v]
                mt = -(-m // vi["bm"])
                if vi["bm"] > 2 * max(16, m) and vi["bm"] > 32:
                    continue  # a tile far taller than M only wastes MFMA work
                for sp in SPLITS:
                    tiles = mt * -(-n // vi["bn"])
                    if sp > 1 and tiles >= 256:
                        continue
                    if sp > kk // 256:
                        continue
                    k.gemm.force(v, sp)
                    rows.append((timeit(), v, sp))
            k.gemm.force(None)
            rows.sort()
            t, v, sp = pick(rows, m, n)
            plan = k.gemm.plan(m, n, kk, epi)
            t_plan = timeit()  # unforced: the planner's own choice (the streaming kernel included)
            fl = 2.0 * m * n * kk
            rec = {"k": kk, "n": n, "m": m, "epi": int(epi), "best": [v, sp, round(t, 2)],
                   "planner": [plan["variant"], plan["splits"], round(t_plan, 2)],
                   "tflops_best": round(fl / t / 1e6, 1), "top": [[round(a, 2), b, c] for a, b, c in rows[:6]]}
            results.append(rec)
            print(json.dumps(rec), flush=True)
    os.makedirs(os.path.dirname(args.out) or ".", exist_ok=True)
    with open(args.out, "w") as f:
        json.dump({"device": "MI355X", "variants": variants(), "results": results,
                   "seconds": round(time.time() - t_start, 1)}, f, indent=1)
    print("// measured table rows: {k, n, m, variant, splits}", file=sys.stderr)
    for r in results:
        print(f"    {{{r['k']}, {r['n']}, {r['m']}, {r['best'][0]}, {r['best'][1]}}},", file=sys.stderr)


if __name__ == "__main__":
    main()
