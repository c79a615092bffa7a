/*
 * oracle.c — CPU restatement of decide's reference arithmetic for the prefill
 * GEMM path. TEST INFRASTRUCTURE ONLY: the checker that tests/, the smoke
 * check and bench.py's cpu_baseline leg compare the HIP library against. The
 * product (decide_amd/) never links, loads or calls it.
 *
 * Each function cites the decide source it restates (paths relative to the
 * decide tree). Pinning (how each function is checked independently of this
 * file — see tests/test_oracle.py):
 *   orc_gemm_nt          KAT + brute force vs numpy float64 matmul (golden fixtures),
 *                        exact integer closed form, one-hot rows, linearity.
 *   orc_swiglu_interleaved  decide's KAT swiglu_pairs_blocks (cpu_ref.rs:212-221)
 *                        plus a closed form on a 64-column row.
 *   orc_rmsnorm          decide's KAT rmsnorm_by_hand (cpu_ref.rs:204-210) plus
 *                        scale invariance.
 *   orc_final_head       composition of rmsnorm and a dot product, checked
 *                        against numpy float64 on golden fixtures.
 *   orc_f16_from_f32 / orc_bf16_from_f32 / orc_f16_to_f32
 *                        numpy float16 (IEEE RNE) on every f16 bit pattern and
 *                        on a sweep of f32 values; bf16 against a bit-level
 *                        closed form.
 *   orc_interleave_gate_up / orc_deinterleave_q_gate
 *                        hand-written permutation KATs.
 *   orc_gemm_f32_fast    agrees with orc_gemm_nt within fp32 rounding.
 *   orc_fill_normal      the library's own seeded Gaussian (not a decide
 *                        function: it makes the random-init weights), restated
 *                        so the host can rebuild a random-init model bit for bit;
 *                        checked bitwise against a numpy float32 restatement,
 *                        against float64 Box–Muller (math.log/cos/sin) within
 *                        fp32 rounding, and by its moments.
 * Build: oracle/Makefile (gcc -O2 -fopenmp, no -ffast-math: sums stay in order).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------- fp16 / bf16 rounding (the `half` crate 2.7.1 semantics: IEEE
 * round-to-nearest-even; testutil.rs:10-12 rounds inputs through them) ---------- */

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* binary16 bits → float, exact. */
float orc_f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    /* zero or subnormal: m · 2^-24 */
    const float v = (float)m * (1.0f / 16777216.0f);
    return s ? -v : v;
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112u) << 23) | (m << 13));
}

/* float → binary16 bits, round to nearest even, computed on the value (not
 * the bit pattern): pick the two neighbouring representable halves and round. */
uint16_t orc_f16_from_f32(float f) {
  const uint16_t sign = (f2u(f) >> 16) & 0x8000u;
  if (isnan(f)) return (uint16_t)(sign | 0x7e00u);
  double a = fabs((double)f);
  if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u);
  /* quantum: 2^-24 below 2^-14, else 2^(floor(log2 a) - 10) */
  double q;
  if (a < 6.103515625e-05) {
    q = 5.9604644775390625e-08;
  } else {
    int ex;
    frexp(a, &ex); /* a = fr · 2^ex, fr in [0.5, 1) */
    q = ldexp(1.0, ex - 1 - 10);
  }
  double n = floor(a / q);
  const double rem = a - n * q;
  if (rem > 0.5 * q || (rem == 0.5 * q && fmod(n, 2.0) != 0.0)) n += 1.0;
  const double v = n * q; /* exact in double */
  /* encode v */
  uint16_t bits;
  if (v < 6.103515625e-05) {
    bits = (uint16_t)(v / 5.9604644775390625e-08);
  } else {
    int ex;
    const double fr = frexp(v, &ex);                  /* v = fr·2^ex */
    const uint32_t e16 = (uint32_t)(ex - 1 + 15);      /* biased */
    const uint32_t m16 = (uint32_t)((fr * 2.0 - 1.0) * 1024.0);
    bits = (uint16_t)((e16 << 10) | m16);
  }
  return (uint16_t)(sign | bits);
}

float orc_f16_round(float f) { return orc_f16_to_f32(orc_f16_from_f32(f)); }

uint16_t orc_bf16_from_f32(float f) {
  const uint32_t u = f2u(f);
  if (isnan(f)) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

void orc_f16_array_to_f32(const uint16_t* h, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(h[i]);
}
void orc_f32_array_to_f16(const float* f, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f16_from_f32(f[i]);
}

/* ---------- math helpers (cpu_ref.rs:6-8) ---------- */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ---------- GEMM (cpu_ref.rs:24-35) ----------
 * y[i][j] = Σ_k x[i][k]·w[j][k], each product widened to f64 and summed in
 * k order in f64, stored as f32. Inputs are fp16 bit patterns (exactly the
 * values the GPU reads), with row strides; y is fp32 [rows, n], row stride ldy.
 * `rows` (optional) selects which rows of x to compute (row i of y is x row
 * rows[i]); NULL means rows 0..m-1.
 * Blocked for speed without changing any result: threads take 16-column
 * blocks of W (transposed once into a per-thread buffer that stays in cache)
 * and walk the rows four at a time, 4 x 4 outputs per pass over k. Every
 * output is still its own f64 running sum in k order over exact products
 * (fp16 x fp16 fits a double), so the bits do not depend on the blocking or
 * the thread count. */
enum { ORC_JB = 16, ORC_IB = 4 };
void orc_gemm_nt_f16(const uint16_t* x, uint32_t ldx, const uint16_t* w, uint32_t ldw, float* y, uint32_t ldy,
                     uint32_t m, uint32_t n, uint32_t k, const uint32_t* rows, int threads) {
  float* xf = (float*)malloc(((size_t)m * k + 1) * sizeof(float));
  for (size_t i = 0; i < m; ++i) {
    const size_t src = rows ? rows[i] : i;
    for (size_t kk = 0; kk < k; ++kk) xf[i * k + kk] = orc_f16_to_f32(x[src * ldx + kk]);
  }
  const int64_t nblk = ((int64_t)n + ORC_JB - 1) / ORC_JB;
#ifdef _OPENMP
  if (threads < 1) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
  {
    double* wt = (double*)malloc(((size_t)k * ORC_JB + 1) * sizeof(double));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int64_t b = 0; b < nblk; ++b) {
      const size_t j0 = (size_t)b * ORC_JB, jn = n - j0 < ORC_JB ? n - j0 : ORC_JB;
      for (size_t kk = 0; kk < k; ++kk)
        for (size_t c = 0; c < ORC_JB; ++c)  /* columns past n repeat the last one (never stored) */
          wt[kk * ORC_JB + c] = orc_f16_to_f32(w[(j0 + (c < jn ? c : jn - 1)) * (size_t)ldw + kk]);
      for (size_t i0 = 0; i0 < m; i0 += ORC_IB) {
        const size_t in = m - i0 < ORC_IB ? m - i0 : ORC_IB;
        const float* xr[ORC_IB];
        for (size_t r = 0; r < ORC_IB; ++r) xr[r] = xf + (i0 + (r < in ? r : in - 1)) * k;
        for (size_t c0 = 0; c0 < jn; c0 += 4) {
          double a[ORC_IB][4] = {{0}};
          for (size_t kk = 0; kk < k; ++kk) {
            const double* w4 = wt + kk * ORC_JB + c0;
            for (size_t r = 0; r < ORC_IB; ++r) {
              const double xv = xr[r][kk];
              for (size_t c = 0; c < 4; ++c) a[r][c] += xv * w4[c];
            }
          }
          for (size_t r = 0; r < in; ++r)
            for (size_t c = 0; c < 4 && c0 + c < jn; ++c) y[(i0 + r) * (size_t)ldy + j0 + c0 + c] = (float)a[r][c];
        }
      }
    }
    free(wt);
  }
  free(xf);
}

/* Same on f32 inputs (cpu_ref::gemm_nt's own signature). */
void orc_gemm_nt(const float* x, const float* w, float* y, uint32_t m, uint32_t n, uint32_t k) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      double a = 0;
      for (size_t kk = 0; kk < k; ++kk) a += (double)x[i * k + kk] * (double)w[j * k + kk];
      y[i * n + j] = (float)a;
    }
}

/* ---------- SwiGLU over the 16-column interleave (cpu_ref.rs:37-50) ---------- */
void orc_swiglu_interleaved(const float* y, float* out, uint32_t m, uint32_t n2, uint32_t blk) {
  const uint32_t n = n2 / 2;
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      const size_t b = j / blk, wv = j % blk;
      const float g = y[i * n2 + b * 2 * blk + wv];
      const float u = y[i * n2 + b * 2 * blk + blk + wv];
      out[i * n + j] = orc_silu(g) * u;
    }
}

/* ---------- RMSNorm (cpu_ref.rs:10-22) ---------- */
void orc_rmsnorm(const float* x, const float* w, float* out, uint32_t rows, uint32_t h, int add_one, float eps) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = x + r * h;
    double ss = 0;
    for (size_t i = 0; i < h; ++i) ss += (double)row[i] * (double)row[i];
    const double ms = ss / (double)h;
    const float inv = 1.0f / sqrtf((float)ms + eps);
    for (size_t i = 0; i < h; ++i) {
      const float wv = add_one ? 1.0f + w[i] : w[i];
      out[r * h + i] = row[i] * inv * wv;
    }
  }
}

/* ---------- candidate head (cpu_ref.rs:190-198; head.metal:30-59) ----------
 * logits[r*max_cand + c] = Σ_i norm(x_r)[i] · bf16(table[cand[r*max_cand+c]][i]),
 * f64 sum, for c < min(ncand[r], max_cand). */
void orc_final_head(const float* x, const float* w, const uint16_t* table, const uint32_t* cand,
                    const uint32_t* ncand, float* logits, uint32_t rows, uint32_t hidden, uint32_t max_cand,
                    float eps) {
  float* hn = (float*)malloc((size_t)hidden * sizeof(float));
  for (size_t r = 0; r < rows; ++r) {
    orc_rmsnorm(x + r * hidden, w, hn, 1, hidden, 1, eps);
    const uint32_t n = ncand[r] < max_cand ? ncand[r] : max_cand;
    for (size_t c = 0; c < n; ++c) {
      const uint16_t* e = table + (size_t)cand[r * max_cand + c] * hidden;
      double a = 0;
      for (size_t i = 0; i < hidden; ++i) a += (double)hn[i] * (double)orc_bf16_to_f32(e[i]);
      logits[r * max_cand + c] = (float)a;
    }
  }
  free(hn);
}

/* ---------- weight layouts (convert.rs:37-62) ---------- */
void orc_interleave_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint32_t n, uint32_t k,
                            uint32_t block) {
  size_t o = 0;
  for (size_t b = 0; b < n / block; ++b) {
    for (size_t r = 0; r < block; ++r, o += k) memcpy(out + o, gate + (b * block + r) * k, k * 2);
    for (size_t r = 0; r < block; ++r, o += k) memcpy(out + o, up + (b * block + r) * k, k * 2);
  }
}

void orc_deinterleave_q_gate(const uint16_t* src, uint16_t* out, uint32_t heads, uint32_t head_dim, uint32_t k) {
  size_t o = 0;
  for (size_t part = 0; part < 2; ++part)
    for (size_t h = 0; h < heads; ++h)
      for (size_t d = 0; d < head_dim; ++d, o += k) memcpy(out + o, src + ((h * 2 + part) * head_dim + d) * k, k * 2);
}

/* ---------- fast CPU fp32 GEMM (the timed baseline, not a parity oracle) ----------
 * y[m][n] = Σ_k x[m][k]·w[n][k] in fp32, blocked, OpenMP over n-blocks. */
void orc_gemm_f32_fast(const float* x, const float* w, float* y, uint32_t m, uint32_t n, uint32_t k, int threads) {
#ifdef _OPENMP
  if (threads < 1) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
  for (int64_t jb = 0; jb < (int64_t)n; jb += 8) {
    const size_t j1 = (size_t)jb + 8 < n ? (size_t)jb + 8 : n;
    for (size_t i = 0; i < m; ++i) {
      const float* xr = x + i * k;
      for (size_t j = (size_t)jb; j < j1; ++j) {
        const float* wr = w + j * k;
        float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        size_t kk = 0;
        for (; kk + 8 <= k; kk += 8)
          for (int q = 0; q < 8; ++q) a[q] += xr[kk + q] * wr[kk + q];
        float s = 0;
        for (int q = 0; q < 8; ++q) s += a[q];
        for (; kk < k; ++kk) s += xr[kk] * wr[kk];
        y[i * n + j] = s;
      }
    }
  }
}

/* ---------- metrics (testutil.rs:14-39 semantics) ---------- */
/* relative Frobenius error ‖got − want‖ / ‖want‖ in f64 */
double orc_rel_frobenius(const float* got, const float* want, size_t n) {
  double num = 0, den = 0;
  for (size_t i = 0; i < n; ++i) {
    const double d = (double)got[i] - (double)want[i];
    num += d * d;
    den += (double)want[i] * (double)want[i];
  }
  return den > 0 ? sqrt(num / den) : sqrt(num);
}

/* index of the worst violation of |g − w| <= atol + rtol·|w| (NaN fails), or -1 */
int64_t orc_assert_close(const float* got, const float* want, size_t n, float atol, float rtol) {
  int64_t worst = -1;
  float worst_over = 0;
  for (size_t i = 0; i < n; ++i) {
    const float err = fabsf(got[i] - want[i]), tol = atol + rtol * fabsf(want[i]);
    const float over = err - tol;
    if (!(over <= 0.0f) && (worst < 0 || !(over <= worst_over))) {
      worst = (int64_t)i;
      worst_over = over;
    }
  }
  return worst;
}

/* ---------- seeded Gaussian: the library's random-init generator, restated ----------
 * Element i of the stream with seed s (decide_amd/csrc/normal_gen.h states the
 * same steps for the device): two 24-bit uniforms a, b from splitmix64's
 * finaliser over s + φ(2p+1) and s + φ(2p+2), p = i/2; Box–Muller with
 * r = sqrt(−2 ln u1), u1 = (a + ½)·2⁻²⁴, and θ = 2π(b + ½)·2⁻²⁴ = (π/4)(o + t)
 * (octant o = b's top 3 bits, t from the other 21); even i: r·cos θ, odd i:
 * r·sin θ; value = (r·trig)·sd + mean, then RNE to the tensor's type.
 * Only IEEE-rounded fp32 +, −, ×, ÷ and sqrt, in this order, no contraction
 * (-ffp-contract=off): ln via the atanh series on m ∈ [√½, √2), sin/cos of
 * (π/4)t via Taylor series; constants are the fp32 roundings of 1/k, ln 2,
 * √2 and ±(π/4)^k/k!. */
static uint64_t nrm_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static float nrm_ln(float u) {
  const uint32_t bits = f2u(u);
  int e = (int)(bits >> 23) - 127;
  float m = u2f((bits & 0x7fffffu) | 0x3f800000u);
  if (m > 0x1.6a09e6p+0f) {
    m = m * 0.5f;
    e = e + 1;
  }
  const float z = (m - 1.0f) / (m + 1.0f);
  const float z2 = z * z;
  float p = 0x1.745d18p-4f;
  p = p * z2 + 0x1.c71c72p-4f;
  p = p * z2 + 0x1.24924ap-3f;
  p = p * z2 + 0x1.99999ap-3f;
  p = p * z2 + 0x1.555556p-2f;
  p = p * z2 + 1.0f;
  return (float)e * 0x1.62e430p-1f + (z + z) * p;
}

static void nrm_sincos(float t, float* s, float* c) {
  const float t2 = t * t;
  float ps = -0x1.e30750p-30f;
  ps = ps * t2 + 0x1.507834p-22f;
  ps = ps * t2 - 0x1.32d2ccp-15f;
  ps = ps * t2 + 0x1.466bc6p-9f;
  ps = ps * t2 - 0x1.4abbcep-4f;
  ps = ps * t2 + 0x1.921fb6p-1f;
  *s = t * ps;
  float pc = 0x1.f9d38ap-34f;
  pc = pc * t2 - 0x1.a6d1f2p-26f;
  pc = pc * t2 + 0x1.e1f506p-19f;
  pc = pc * t2 - 0x1.55d3c8p-12f;
  pc = pc * t2 + 0x1.03c1f0p-6f;
  pc = pc * t2 - 0x1.3bd3ccp-2f;
  *c = pc * t2 + 1.0f;
}

float orc_normal_at(uint64_t seed, uint64_t i, float mean, float sd) {
  const uint64_t p = i >> 1, phi = 0x9e3779b97f4a7c15ull;
  const uint32_t a = (uint32_t)(nrm_mix64(seed + phi * (2 * p + 1)) >> 40);
  const uint32_t b = (uint32_t)(nrm_mix64(seed + phi * (2 * p + 2)) >> 40);
  const float r = sqrtf(-2.0f * nrm_ln(((float)a + 0.5f) * 0x1p-24f));
  const uint32_t o = b >> 21;
  const float t = ((float)(b & 0x1fffffu) + 0.5f) * 0x1p-21f;
  float sb, cb;
  nrm_sincos((o & 1u) ? 1.0f - t : t, &sb, &cb);
  if (o & 1u) sb = -sb;
  /* θ = k·π/2 + β, β = ±(π/4)·(t or 1 − t): rotate (cos β, sin β) by k quarter turns */
  const uint32_t k = ((o + 1u) >> 1) & 3u;
  const float cth = k == 0 ? cb : k == 1 ? -sb : k == 2 ? -cb : sb;
  const float sth = k == 0 ? sb : k == 1 ? cb : k == 2 ? -sb : -cb;
  const float z = r * ((i & 1) ? sth : cth);
  return z * sd + mean;
}

/* n values of the stream into out as fp16 (dtype 0), bf16 (1) or fp32 (2) bits. */
void orc_fill_normal(void* out, uint64_t n, uint64_t seed, float mean, float sd, uint32_t dtype, int threads) {
#ifdef _OPENMP
  if (threads < 1) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static, 65536)
#endif
  for (int64_t ii = 0; ii < (int64_t)n; ++ii) {
    const uint64_t i = (uint64_t)ii;
    const float v = orc_normal_at(seed, i, mean, sd);
    if (dtype == 0)
      ((uint16_t*)out)[i] = orc_f16_from_f32(v);
    else if (dtype == 1)
      ((uint16_t*)out)[i] = orc_bf16_from_f32(v);
    else
      ((float*)out)[i] = v;
  }
}
