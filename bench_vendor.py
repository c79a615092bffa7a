#!/usr/bin/env python3
"""The path's GEMM shapes through the vendor library, for comparison only (not part of the product path).

`torch.matmul` on ROCm dispatches fp16 GEMMs to hipBLASLt. This times Y = X·Wᵀ (plain store epilogue: no
SwiGLU, no residual add) for the shapes decide_amd.shape_report measures with this build's kernels, with
HIP events over 100 launches after 20 warm-ups; for the gate|up shapes also the product followed by the SwiGLU
decide's path takes from it (eager torch: fp32 silu(gate)·up over the 16-column interleave, rounded to fp16).
Interleaved with each (same box, same tensors, same stream), this build's planned kernel for the shape with the
epilogue decide's path runs (C1 StoreF32, gate|up SwiGLU, down the residual add), by the same events: two rounds
per shape, reported as `this_build_event_us`. The kernel each shape runs, and its own duration, come from
running this module under the profiler:

    rocprofv3 --kernel-trace --stats -d gpurun_out/blas -o mm --output-format csv -- python3 bench_vendor.py
"""

from __future__ import annotations

import json

SHAPES = [  # (name, M, N, K) — BASELINE's C1, the C2 MLP pair and the C4 gate|up
    ("C1 proj", 276, 9216, 2560),
    ("C2 gate|up", 603, 18432, 2560),
    ("C2 down", 603, 2560, 9216),
    ("C4 gate|up", 2307, 18432, 2560),
]


def _this_build(kernels, x, w, name: str, m: int, n: int, k: int, launches: int = 100) -> float:
    """Mean µs per launch of this build's planned kernel on the same tensors, with the path's epilogue."""
    import torch

    from decide_amd.kernels import Epilogue

    epi = Epilogue.SwigluF16 if "gate|up" in name else Epilogue.AddF32 if "down" in name else Epilogue.StoreF32
    cols = n // 2 if epi == Epilogue.SwigluF16 else n
    y = torch.zeros(m, cols, device="cuda", dtype=torch.float16 if epi == Epilogue.SwigluF16 else torch.float32)
    s = torch.cuda.current_stream().cuda_stream

    def run():
        kernels.gemm.gemm(s, (x, 0), (w, 0), (y, 0), m, n, k, k, k, cols, epi)

    for _ in range(20):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(launches):
        run()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / launches * 1e3


def main() -> None:
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("no GPU")
    from decide_amd.kernels import Kernels

    kernels = Kernels()
    torch.manual_seed(0)
    for name, m, n, k in SHAPES:
        x = torch.randn(m, k, device="cuda", dtype=torch.float16)
        w = torch.randn(n, k, device="cuda", dtype=torch.float16) * 0.02
        for _ in range(20):
            y = x @ w.t()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(100):
            y = x @ w.t()
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) / 100 * 1e3
        rec = {"shape": name, "m": m, "n": n, "k": k, "event_us": round(us, 2),
               "tflops": round(2.0 * m * n * k / us / 1e6, 1)}
        if "gate|up" in name:
            # what decide's path needs from this product: silu(gate) * up over the 16-column interleave, in fp32,
            # rounded to fp16 (this build fuses it into the GEMM's epilogue; here it is eager torch after it)
            def swiglu(y):
                v = y.view(m, n // 32, 2, 16).float()
                return (torch.nn.functional.silu(v[:, :, 0]) * v[:, :, 1]).half()
            for _ in range(5):
                o = swiglu(x @ w.t())
            torch.cuda.synchronize()
            e0.record()
            for _ in range(50):
                o = swiglu(x @ w.t())
            e1.record()
            e1.synchronize()
            rec["with_swiglu_event_us"] = round(e0.elapsed_time(e1) / 50 * 1e3, 2)
            del o
        # interleaved: this build, the library again, this build again
        ours = [_this_build(kernels, x, w, name, m, n, k)]
        e0.record()
        for _ in range(100):
            y = x @ w.t()
        e1.record()
        e1.synchronize()
        rec["event_us_second_round"] = round(e0.elapsed_time(e1) / 100 * 1e3, 2)
        ours.append(_this_build(kernels, x, w, name, m, n, k))
        rec["this_build_event_us"] = [round(v, 2) for v in ours]
        print(json.dumps(rec), flush=True)
        del y


if __name__ == "__main__":
    main()
