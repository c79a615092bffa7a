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
