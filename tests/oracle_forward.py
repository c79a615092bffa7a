"""The oracle's hybrid decoder forward: decide's layer order and fp16 rounding points
(forward.rs:1125-1310; Buffers, forward.rs:124-180) strung from the oracle's pieces (cpu_ref.rs).
Test infrastructure only.

Rounding points as in decide: h, g, mlp, qo and the K/V caches are fp16; p, x, q, k, v, o and the
recurrent state are fp32. Every GEMM is cpu_ref::gemm_nt (f64 sums) on the fp16 operands.
"""

from __future__ import annotations

import numpy as np

import oracle_lib as orc

HIDDEN = 2560
INTER = 9216
LIN_Z, LIN_B, LIN_A = 8192, 12288, 12320
Q_DIM, KV_DIM, ATT_K, ATT_V = 4096, 1024, 8192, 9216
NV, DV, DK = 32, 128, 128


def _f16(a: np.ndarray) -> np.ndarray:
    return orc.f16_round(a).astype(np.float16)


def _norm16(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    return _f16(orc.rmsnorm(x, w, add_one=True))


def _rope_heads(p: np.ndarray, col: int, heads: int, w: np.ndarray, pos: np.ndarray) -> np.ndarray:
    """head_norm_rope of `heads` 256-dim heads starting at column `col` of each row → fp16 [rows, heads, 256]."""
    out = np.empty((p.shape[0], heads, 256), np.float32)
    for r in range(p.shape[0]):
        for h in range(heads):
            out[r, h] = orc.head_norm_rope(p[r, col + 256 * h:col + 256 * (h + 1)], w, int(pos[r]))
    return _f16(out)


def _mlp(W, pre, x, gemm):
    h = _norm16(x, W[pre + "post_norm"])
    mlp = _f16(orc.swiglu_interleaved(gemm(h, W[pre + "w_gu"])))
    return x + gemm(mlp, W[pre + "w_down"])


def forward(W: dict, layers: int, ids: np.ndarray, ans_rows: np.ndarray, cand: np.ndarray, ncand: np.ndarray,
            max_cand: int, prune: bool = True, gemm=None) -> np.ndarray:
    """Candidate logits [n_ans, max_cand] (NaN where not written) for a full-route forward from position 0.

    W maps decide-weights-v1 names to arrays: fp16 GEMM weights [N, K], fp32 small parameters, and the
    embedding as raw bf16 bits [vocab, 2560]. ``gemm(x, w)`` computes every projection: by default
    cpu_ref::gemm_nt on the fp16 operands (f64 sums); another correct implementation may be passed."""
    gemm = gemm or orc.gemm_nt_f16
    t = len(ids)
    pos = np.arange(t, dtype=np.uint32)
    x = orc.embed_bf16(ids, W["embed"])
    xs = None
    for l in range(layers):
        pre = f"L{l}."
        attn = (l + 1) % 4 == 0
        h = _norm16(x, W[pre + "in_norm"])
        if not attn:
            p = gemm(h, W[pre + "w_in"])
            q, k, v = orc.conv_silu_l2(p, t, np.zeros((3, orc.CONV_DIM), np.float32), W[pre + "conv_w"])
            o, _ = orc.gated_delta(q, k, v, p[:, LIN_A:LIN_A + NV], p[:, LIN_B:LIN_B + NV], W[pre + "a_log"],
                                   W[pre + "dt_bias"], np.zeros((NV, DV, DK), np.float32), t)
            g = _f16(orc.gated_rmsnorm_silu(o, p[:, LIN_Z:LIN_Z + Q_DIM], W[pre + "gnorm"], t))
        elif prune and l == layers - 1:
            w_in = W[pre + "w_in"]
            pkv = gemm(h, w_in[ATT_K:])
            kc = _rope_heads(pkv, 0, 4, W[pre + "k_norm"], pos)
            vc = _f16(pkv[:, KV_DIM:].reshape(t, 4, 256))
            ps = gemm(h[ans_rows], w_in[:ATT_K])
            qo = _rope_heads(ps, 0, 16, W[pre + "q_norm"], ans_rows)
            g = _f16(orc.attention(qo.astype(np.float32), ans_rows, kc.astype(np.float32), vc.astype(np.float32),
                                   ps[:, Q_DIM:]))
            xs = x[ans_rows] + gemm(g, W[pre + "w_out"])
            xs = _mlp(W, pre, xs, gemm)
            break
        else:
            p = gemm(h, W[pre + "w_in"])
            qo = _rope_heads(p, 0, 16, W[pre + "q_norm"], pos)
            kc = _rope_heads(p, ATT_K, 4, W[pre + "k_norm"], pos)
            vc = _f16(p[:, ATT_V:ATT_V + KV_DIM].reshape(t, 4, 256))
            g = _f16(orc.attention(qo.astype(np.float32), pos, kc.astype(np.float32), vc.astype(np.float32),
                                   p[:, Q_DIM:]))
        x = x + gemm(g, W[pre + "w_out"])
        x = _mlp(W, pre, x, gemm)
    if xs is None:
        xs = x[ans_rows]
    return orc.final_head(xs, W["final_norm"], W["embed"], cand, ncand, max_cand)


# ---- random-init models rebuilt on the host ----------------------------------------------------------------------
# dh_model_init_random(seed) fills tensor i of the model's registry with the stream
# seed + φ·(i + 1) (mod 2^64) of the library's seeded Gaussian, which orc_fill_normal restates bit for bit.
PHI = 0x9E3779B97F4A7C15
F16, BF16, F32 = 0, 1, 2


def random_init_registry(layers: int, vocab: int) -> list[tuple[str, tuple, int, float, float]]:
    """(name, shape, dtype code, mean, std) in dh_model_create's registration order: embed, final_norm, then per
    layer in_norm, the mixer's tensors (attention: w_in, q_norm, k_norm, w_out; Gated-DeltaNet: w_in, conv_w, a_log,
    dt_bias, gnorm, w_out), post_norm, w_gu, w_down. Shapes are the [N, K] GEMM layouts."""
    reg = [("embed", (vocab, HIDDEN), BF16, 0.0, 0.02), ("final_norm", (HIDDEN,), F32, 0.0, 0.02)]
    for l in range(layers):
        pre = f"L{l}."
        reg.append((pre + "in_norm", (HIDDEN,), F32, 0.0, 0.02))
        if (l + 1) % 4 == 0:
            reg += [(pre + "w_in", (ATT_V + KV_DIM, HIDDEN), F16, 0.0, 0.02), (pre + "q_norm", (256,), F32, 0.0, 0.02),
                    (pre + "k_norm", (256,), F32, 0.0, 0.02), (pre + "w_out", (HIDDEN, Q_DIM), F16, 0.0, 0.02)]
        else:
            reg += [(pre + "w_in", (LIN_A + NV, HIDDEN), F16, 0.0, 0.02),
                    (pre + "conv_w", (orc.CONV_DIM, 4), F32, 0.0, 0.3), (pre + "a_log", (NV,), F32, 0.5, 0.5),
                    (pre + "dt_bias", (NV,), F32, 0.0, 0.5), (pre + "gnorm", (DV,), F32, 1.0, 0.02),
                    (pre + "w_out", (HIDDEN, NV * DV), F16, 0.0, 0.02)]
        reg += [(pre + "post_norm", (HIDDEN,), F32, 0.0, 0.02), (pre + "w_gu", (2 * INTER, HIDDEN), F16, 0.0, 0.02),
                (pre + "w_down", (HIDDEN, INTER), F16, 0.0, 0.02)]
    return reg


def random_init_tensor(seed: int, index: int, shape, dtype: int, mean: float, std: float) -> np.ndarray:
    """Tensor `index` of a model after dh_model_init_random(seed), as forward() takes it (bf16 as raw bits)."""
    n = int(np.prod(shape))
    return orc.fill_normal(n, (seed + PHI * (index + 1)) % 2**64, mean, std, dtype).reshape(shape)


class RandomInitWeights:
    """The weights of dh_model_init_random(seed) for a (layers, vocab) model, generated on first use. Keeps the
    embedding and the most recent `keep` other tensors, so a deep forward needs about one layer's weights at once."""

    def __init__(self, seed: int, layers: int, vocab: int, keep: int = 12):
        self.seed = seed
        self.reg = {name: (i, shape, dt, mean, std)
                    for i, (name, shape, dt, mean, std) in enumerate(random_init_registry(layers, vocab))}
        self.keep = keep
        self.cache: dict[str, np.ndarray] = {}

    def __getitem__(self, name: str) -> np.ndarray:
        if name not in self.cache:
            i, shape, dt, mean, std = self.reg[name]
            others = [k for k in self.cache if k != "embed"]
            if len(others) >= self.keep:
                del self.cache[others[0]]
            self.cache[name] = random_init_tensor(self.seed, i, shape, dt, mean, std)
        return self.cache[name]
