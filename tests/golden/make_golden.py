"""Writes the small golden fixtures under tests/golden/ with numpy float64.

These pin the CPU oracle (tests/test_oracle.py) with a library routine that
shares no code with it: numpy's float64 matmul for the GEMM, float64 numpy
for SwiGLU and the candidate head. decide ships no GEMM vectors of its own
(its GPU kernel tests are not in the snapshot), so these are the GEMM path's
golden vectors. Run: python tests/golden/make_golden.py
"""

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def silu64(x):
    return x / (1.0 + np.exp(-x))


def swiglu64(y, blk=16):
    m, n2 = y.shape
    out = np.empty((m, n2 // 2))
    for j in range(n2 // 2):
        b, w = divmod(j, blk)
        out[:, j] = silu64(y[:, b * 2 * blk + w]) * y[:, b * 2 * blk + blk + w]
    return out


def bf16_bits(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def main():
    rng = np.random.default_rng(0xDEC1DE)
    index = {"gemm": []}
    for (m, n, k, swiglu) in [(1, 32, 32, False), (7, 64, 96, True), (17, 32, 64, False), (33, 96, 160, True),
                              (24, 64, 2560, False), (5, 128, 320, True)]:
        x = rng.standard_normal((m, k)).astype(np.float16)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
        y = x.astype(np.float64) @ w.astype(np.float64).T
        arrays = {"x": x, "w": w, "y": y.astype(np.float32)}
        if swiglu:
            arrays["swiglu"] = swiglu64(y.astype(np.float32).astype(np.float64)).astype(np.float32)
        name = f"gemm_m{m}_n{n}_k{k}.npz"
        np.savez_compressed(os.path.join(HERE, name), **arrays)
        index["gemm"].append({"file": name, "m": m, "n": n, "k": k, "swiglu": swiglu})

    # candidate head: 6 rows, hidden 256, vocab 1000, max_cand 8, ragged counts (0, > max)
    rows, hidden, vocab, max_cand = 6, 256, 1000, 8
    x = rng.standard_normal((rows, hidden)).astype(np.float32) * 3
    w = (rng.standard_normal(hidden) * 0.02).astype(np.float32)
    table = bf16_bits(rng.standard_normal((vocab, hidden)) * 0.02)
    cand = rng.integers(0, vocab, (rows, max_cand)).astype(np.uint32)
    ncand = np.array([8, 3, 0, 1, 12, 5], dtype=np.uint32)
    t32 = (table.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    logits = np.full((rows, max_cand), np.nan, dtype=np.float32)
    for r in range(rows):
        xr = x[r].astype(np.float64)
        inv = 1.0 / np.sqrt(np.mean(xr * xr) + 1e-6)
        hn = xr * inv * (1.0 + w.astype(np.float64))
        for c in range(min(int(ncand[r]), max_cand)):
            logits[r, c] = hn @ t32[cand[r, c]]
    np.savez_compressed(os.path.join(HERE, "head_small.npz"), x=x, w=w, table=table, cand=cand, ncand=ncand,
                        logits=logits, max_cand=np.array(max_cand))
    index["head"] = [{"file": "head_small.npz"}]
    with open(os.path.join(HERE, "index.json"), "w") as f:
        json.dump(index, f, indent=1)


if __name__ == "__main__":
    main()
