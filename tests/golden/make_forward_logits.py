"""Writes the oracle's candidate logits for two whole-model forwards, on models that dh_model_init_random(0xDEC1DE)
makes, rebuilt on the host bit for bit (oracle_forward.RandomInitWeights):

  c5     -> tests/golden/c5_full_logits.npz: BASELINE config 5 at its stated shape (36 layers, T = 2,307,
            vocab 151,936, 3 answers x 8 candidates, one list ragged);
  ref603 -> tests/golden/ref603_logits.npz: decide's own model shape (32 layers, vocab 248,320; config.rs:5, 32)
            on a ticket-like request (603 tokens after a 107-token prefix, 6 answers with 2..62 candidates;
            README.md:17-20).

Each holds two oracle forwards over the whole sequence from position 0 (tests/oracle_forward.py: decide's layer
order and rounding points, forward.rs:1118-1310):
  * logits_f64: every projection is cpu_ref::gemm_nt (f64 sums of exact products, cpu_ref.rs:24-35) — the oracle;
  * logits_f32sum: the same forward with the GEMM sums in fp32 (orc_gemm_f32_fast) — a second correct fp32
    implementation, whose distance from the first is the fp32 noise floor at that shape.
CPU only (c5 about 25 minutes on 8 cores, ref603 about 8). Run from the repository root:
    python tests/golden/make_forward_logits.py c5|ref603
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.dirname(HERE)]

import oracle_forward  # noqa: E402
import oracle_lib as orc  # noqa: E402
from decide_amd import synth  # noqa: E402

INIT_SEED = 0xDEC1DE


def request_c5(t: int = 2307, vocab: int = 151936, seed: int = 5300, answers: int = 3, cands: int = 8):
    """Token ids, answer rows, candidate ids and candidate counts of the config-5 request (ragged second list)."""
    ids = synth.uniform_ids(synth.seed_for(seed), t, vocab).astype(np.uint32)
    ans = np.array([t // 3, (2 * t) // 3, t - 1], np.uint32)[:answers]
    cand = synth.uniform_ids(synth.seed_for(seed + 1), answers * cands, vocab).astype(np.uint32).reshape(answers, cands)
    ncand = np.full(answers, cands, np.uint32)
    ncand[1] = cands - 2
    return ids, ans, cand, ncand


REF_PREFIX, REF_VOCAB, REF_MAX_CAND = 107, 248320, 62
REF_NCAND = (2, 4, 8, 16, 30, 62)


def request_ref(t: int, n_answers: int, seed: int = 6100):
    """A request shaped like decide's (README.md:17-20): the same 107-token prefix for every length, then the
    state and questions; answers in the last rows, each with its own candidate count (2..62)."""
    prefix = synth.uniform_ids(synth.seed_for(6000), REF_PREFIX, REF_VOCAB).astype(np.uint32)
    rest = synth.uniform_ids(synth.seed_for(seed + t), t - REF_PREFIX, REF_VOCAB).astype(np.uint32)
    ids = np.concatenate([prefix, rest])
    ans = np.array([t - 1 - 9 * (n_answers - 1 - i) for i in range(n_answers)], np.uint32)
    cand = synth.uniform_ids(synth.seed_for(seed + t + 1), n_answers * REF_MAX_CAND, REF_VOCAB).astype(np.uint32)
    cand = cand.reshape(n_answers, REF_MAX_CAND)
    ncand = np.array([REF_NCAND[i % len(REF_NCAND)] for i in range(n_answers)], np.uint32)
    return ids, ans, cand, ncand


CONFIGS = {
    # name: (layers, vocab, max_cand, request, output file)
    "c5": (36, 151936, 8, lambda: request_c5(), "c5_full_logits.npz"),
    "ref603": (32, REF_VOCAB, REF_MAX_CAND, lambda: request_ref(603, 6), "ref603_logits.npz"),
}


def gemm_fp32_sums(x, w):
    return orc.gemm_f32_fast(np.asarray(x, np.float16).astype(np.float32), np.asarray(w, np.float16).astype(np.float32))


class _Progress:
    """Wraps a GEMM to print one line per layer (every layer calls its in-projection first)."""

    def __init__(self, gemm, label):
        self.gemm, self.label, self.calls, self.t0 = gemm, label, 0, time.time()

    def __call__(self, x, w):
        self.calls += 1
        if w.shape[0] in (10240, 12352, 2048):  # an in-projection (or the pruned layer's k|v): a new layer
            print(f"[{self.label}] gemm {self.calls}, {time.time() - self.t0:.0f} s", flush=True)
        return self.gemm(x, w)


def main(name: str) -> None:
    layers, vocab, max_cand, make_request, fname = CONFIGS[name]
    ids, ans, cand, ncand = make_request()
    out = {"ids": ids, "ans": ans, "cand": cand, "ncand": ncand,
           "meta": np.array([layers, len(ids), vocab, len(ans), max_cand, INIT_SEED], np.uint64)}
    for key, gemm in (("logits_f64", orc.gemm_nt_f16), ("logits_f32sum", gemm_fp32_sums)):
        W = oracle_forward.RandomInitWeights(INIT_SEED, layers, vocab)
        t0 = time.time()
        out[key] = oracle_forward.forward(W, layers, ids, ans, cand, ncand, max_cand, prune=True,
                                          gemm=_Progress(gemm, key))
        print(f"{key}: {time.time() - t0:.0f} s", flush=True)
    w = ~np.isnan(out["logits_f64"])
    floor = float(np.abs(out["logits_f32sum"][w] - out["logits_f64"][w]).max())
    print(f"fp32-sum oracle vs f64 oracle: max |Δlogit| {floor:.4f}; logits up to {np.abs(out['logits_f64'][w]).max():.3g}")
    path = os.path.join(HERE, fname)
    np.savez_compressed(path, **out)
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "c5")
