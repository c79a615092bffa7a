/*
 * oracle_mixer.c — CPU restatement of decide's reference arithmetic for the
 * non-GEMM parts of the hybrid decoder forward (the Gated-DeltaNet mixer, the
 * gated GQA attention mixer and the embedding gather). TEST INFRASTRUCTURE
 * ONLY, like oracle.c: tests/ and bench.py's cpu_baseline leg use it as the
 * checker; the product never links, loads or calls it.
 *
 * Each function restates one function of crates/decide-engine/src/cpu_ref.rs
 * (cited per function) with the model constants of config.rs:4-41. Where
 * cpu_ref sums in f64 this does too; everything else is f32 in the same
 * order. Pinning (tests/test_oracle_mixer.py):
 *   orc_conv_silu_l2      impulse responses (one-tap kernels reproduce shifted
 *                         rows, through silu), unit norms of q·√128 and k, the
 *                         prev-state rows used for t < 3.
 *   orc_conv_state_update closed form (the last three raw rows) for t ≥ 3,
 *                         t = 1 and t = 2.
 *   orc_gated_delta       closed forms: one token from zero state gives
 *                         o = β·(k·q)·v; β = 0 leaves S decayed by g per step;
 *                         g and β against their formulas at chosen a, b;
 *                         a brute-force numpy recurrence on a tiny head.
 *   orc_gated_rmsnorm_silu hand-computed known answer on a constant segment.
 *   orc_head_norm_rope    position 0 is the plain zero-centred norm; rotation
 *                         preserves each (i, i+32) pair's length; a
 *                         hand-computed angle at position 1.
 *   orc_attention         one visible key returns v·σ(gate); equal scores
 *                         return the mean of v; a numpy float64 softmax.
 *   orc_embed_bf16        bitwise widening of the bf16 rows.
 * Build: oracle/Makefile.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* config.rs:4-31 */
enum {
  NK = 16, DK = 128, NV = 32, DV = 128,
  KEY_DIM = NK * DK, VALUE_DIM = NV * DV, CONV_DIM = 2 * KEY_DIM + VALUE_DIM, CONV_K = 4,
  NQ = 16, NKV = 4, HEAD_DIM = 256, Q_DIM = NQ * HEAD_DIM, KV_DIM = NKV * HEAD_DIM, ROT_DIM = 64
};
static const float EPS = 1e-6f;
static const float ROPE_THETA = 1e7f;

static float silu(float x) { return x / (1.0f + expf(-x)); }                 /* cpu_ref.rs:6 */
static float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }           /* cpu_ref.rs:7 */
static float softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); } /* cpu_ref.rs:8 */

float orc_softplus(float x) { return softplus(x); }

/* config.rs:43-46: inverse frequencies in f32, as HF computes them. */
void orc_inv_freq(float* out) {
  for (int i = 0; i < ROT_DIM / 2; ++i) out[i] = 1.0f / powf(ROPE_THETA, (float)(2 * i) / (float)ROT_DIM);
}

/* cpu_ref.rs:55-81 — causal depthwise conv (kernel 4) + SiLU over the qkv
 * columns of p (row stride ldp), prev = the 3 raw rows before the chunk
 * (oldest first, [3][CONV_DIM]); q = l2norm(q)·DK^-½, k = l2norm(k) per head,
 * v copied. q, k: [t][NK][DK]; v: [t][NV][DV]. */
void orc_conv_silu_l2(const float* p, uint32_t ldp, uint32_t t, const float* prev, const float* w, float* q,
                      float* k, float* v) {
  float* y = (float*)malloc(sizeof(float) * CONV_DIM);
  const float qscale = powf((float)DK, -0.5f);
  for (uint32_t s = 0; s < t; ++s) {
    for (int c = 0; c < CONV_DIM; ++c) {
      double acc = 0.0;
      for (int j = 0; j < CONV_K; ++j) {
        const long src = (long)s - 3 + j;
        const float raw = src >= 0 ? p[(size_t)src * ldp + c] : prev[(size_t)(3 + src) * CONV_DIM + c];
        acc += (double)w[c * CONV_K + j] * (double)raw;
      }
      y[c] = silu((float)acc);
    }
    for (int h = 0; h < 2 * NK; ++h) {
      const float* seg = y + h * DK;
      double ss = 0.0;
      for (int d = 0; d < DK; ++d) ss += (double)seg[d] * (double)seg[d];
      const float inv = 1.0f / sqrtf((float)ss + 1e-6f);
      const float scale = h < NK ? qscale : 1.0f;
      float* dst = h < NK ? q + ((size_t)s * NK + h) * DK : k + ((size_t)s * NK + (h - NK)) * DK;
      for (int d = 0; d < DK; ++d) dst[d] = seg[d] * inv * scale;
    }
    memcpy(v + (size_t)s * VALUE_DIM, y + 2 * KEY_DIM, sizeof(float) * VALUE_DIM);
  }
  free(y);
}

/* cpu_ref.rs:86-95 — the 3 raw qkv rows that end a chunk of t rows. */
void orc_conv_state_update(const float* p, uint32_t ldp, uint32_t t, const float* prev, float* out) {
  for (int i = 0; i < 3; ++i) {
    const long s = (long)t - 3 + i;
    for (int c = 0; c < CONV_DIM; ++c)
      out[(size_t)i * CONV_DIM + c] = s >= 0 ? p[(size_t)s * ldp + c] : prev[(size_t)(3 + s) * CONV_DIM + c];
  }
}

/* cpu_ref.rs:101-129 — sequential gated delta rule; state [NV][DV][DK] in
 * place; a, b rows of stride ldab (value head h at column h); o [t][NV][DV]. */
void orc_gated_delta(const float* q, const float* k, const float* v, const float* a, const float* b, uint32_t ldab,
                     const float* a_log, const float* dt_bias, float* state, uint32_t t, float* o) {
  /* value heads never interact: each runs its own steps (threads split the heads; same arithmetic) */
#pragma omp parallel for schedule(static)
  for (int h = 0; h < NV; ++h) {
    for (uint32_t s = 0; s < t; ++s) {
      const int hk = h / (NV / NK);
      const float g = expf(-(expf(a_log[h])) * softplus(a[(size_t)s * ldab + h] + dt_bias[h]));
      const float beta = sigmoid(b[(size_t)s * ldab + h]);
      const float* kt = k + ((size_t)s * NK + hk) * DK;
      const float* qt = q + ((size_t)s * NK + hk) * DK;
      for (int dv = 0; dv < DV; ++dv) {
        float* row = state + ((size_t)h * DV + dv) * DK;
        double kv = 0.0;
        for (int dk = 0; dk < DK; ++dk) {
          row[dk] *= g;
          kv += (double)row[dk] * (double)kt[dk];
        }
        const float delta = (v[((size_t)s * NV + h) * DV + dv] - (float)kv) * beta;
        double out = 0.0;
        for (int dk = 0; dk < DK; ++dk) {
          row[dk] += kt[dk] * delta;
          out += (double)row[dk] * (double)qt[dk];
        }
        o[((size_t)s * NV + h) * DV + dv] = (float)out;
      }
    }
  }
}

/* cpu_ref.rs:132-145 — per (row, value head): RMSNorm over DV with weight w
 * (no +1), times silu(z); z rows of stride ldz. y [t][VALUE_DIM]. */
void orc_gated_rmsnorm_silu(const float* o, const float* z, uint32_t ldz, const float* w, uint32_t t, float* y) {
  for (uint32_t s = 0; s < t; ++s)
    for (int h = 0; h < NV; ++h) {
      const float* seg = o + ((size_t)s * NV + h) * DV;
      double ms = 0.0;
      for (int d = 0; d < DV; ++d) ms += (double)seg[d] * (double)seg[d];
      ms /= DV;
      const float inv = 1.0f / sqrtf((float)ms + EPS);
      for (int d = 0; d < DV; ++d)
        y[(size_t)s * VALUE_DIM + h * DV + d] = seg[d] * inv * w[d] * silu(z[(size_t)s * ldz + h * DV + d]);
    }
}

/* cpu_ref.rs:149-162 — zero-centred RMSNorm over HEAD_DIM, then RoPE on dims
 * [0, ROT_DIM) at position pos (pairs i, i + 32; f32 angle pos·inv_freq[i],
 * sin/cos evaluated in f64 and rounded). */
void orc_head_norm_rope(const float* seg, const float* w, uint32_t pos, float* out) {
  double ms = 0.0;
  for (int d = 0; d < HEAD_DIM; ++d) ms += (double)seg[d] * (double)seg[d];
  ms /= HEAD_DIM;
  const float inv = 1.0f / sqrtf((float)ms + EPS);
  for (int d = 0; d < HEAD_DIM; ++d) out[d] = seg[d] * inv * (1.0f + w[d]);
  float f[ROT_DIM / 2];
  orc_inv_freq(f);
  for (int i = 0; i < ROT_DIM / 2; ++i) {
    const float ang = (float)pos * f[i];
    const float sn = (float)sin((double)ang), cs = (float)cos((double)ang);
    const float a = out[i], b = out[i + ROT_DIM / 2];
    out[i] = a * cs - b * sn;
    out[i + ROT_DIM / 2] = b * cs + a * sn;
  }
}

/* cpu_ref.rs:167-188 — causal GQA attention for query rows at absolute
 * positions qpos: q [rows][NQ][HEAD_DIM], keys/values [npos][NKV][HEAD_DIM],
 * gate rows of stride ldg (head h, dim d at column h·HEAD_DIM + d); out
 * [rows][Q_DIM] = softmax(q·kᵀ/16)·v ⊙ σ(gate), scores and softmax in f64. */
void orc_attention(const float* q, const uint32_t* qpos, uint32_t rows, const float* kc, const float* vc,
                   const float* gate, uint32_t ldg, float* out) {
#pragma omp parallel for schedule(dynamic)
  for (long s = 0; s < (long)rows; ++s) {
    const uint32_t pos = qpos[s];
    double* sc = (double*)malloc(sizeof(double) * (pos + 1));
    for (int h = 0; h < NQ; ++h) {
      const int kvh = h / (NQ / NKV);
      const float* qv = q + ((size_t)s * NQ + h) * HEAD_DIM;
      double m = -INFINITY;
      for (uint32_t j = 0; j <= pos; ++j) {
        const float* kr = kc + ((size_t)j * NKV + kvh) * HEAD_DIM;
        double acc = 0.0;
        for (int d = 0; d < HEAD_DIM; ++d) acc += (double)qv[d] * (double)kr[d];
        sc[j] = acc / 16.0;
        if (sc[j] > m) m = sc[j];
      }
      double z = 0.0;
      for (uint32_t j = 0; j <= pos; ++j) {
        sc[j] = exp(sc[j] - m);
        z += sc[j];
      }
      for (int d = 0; d < HEAD_DIM; ++d) {
        double acc = 0.0;
        for (uint32_t j = 0; j <= pos; ++j) acc += sc[j] * (double)vc[((size_t)j * NKV + kvh) * HEAD_DIM + d];
        out[(size_t)s * Q_DIM + h * HEAD_DIM + d] =
            (float)(acc / z) * sigmoid(gate[(size_t)s * ldg + h * HEAD_DIM + d]);
      }
    }
    free(sc);
  }
}

/* embed.metal:4-12 / forward.rs:1047-1051 — out[t][c] = float(table[ids[t]][c]), bf16 widened. */
void orc_embed_bf16(const uint32_t* ids, const uint16_t* table, uint32_t t, uint32_t h, float* out) {
  for (uint32_t s = 0; s < t; ++s)
    for (uint32_t c = 0; c < h; ++c) {
      const uint32_t u = (uint32_t)table[(size_t)ids[s] * h + c] << 16;
      memcpy(&out[(size_t)s * h + c], &u, 4);
    }
}
