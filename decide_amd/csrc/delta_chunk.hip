// Chunked gated delta rule for gfx950: the same recurrence as the token-by-
// token kernel (decide: kernels/delta_fast.metal; cpu_ref.rs:101-129),
//   S_t = g_t S_{t-1} + β_t (v_t − g_t S_{t-1} k_t) k_tᵀ,  o_t = S_t q_t,
// rewritten per chunk of C = 64 tokens so that nearly all the work is fp32
// matrix products on v_mfma_f32_16x16x4_f32 (the WY form of the delta rule
// with the decay folded into ratios γ_i/γ_j, γ = cumulative product of g in
// the chunk; every ratio is formed as exp(Lγ_i − Lγ_j) from log-space sums so
// no γ under/overflows):
//   A_ij = β_i (γ_i/γ_j) k_i·k_j (i > j),   T = (I + A)⁻¹,
//   W = T diag(βγ) K,   U = T diag(β) V,   M_ij = (γ_i/γ_j) q_i·k_j (i ≥ j),
// then, in chunk order, with the state S (DV × DK) at the chunk start,
//   V' = U − W Sᵀ,   S ← γ_C S + V'ᵀ diag(γ_C/γ) K,
// and, for every chunk independently once its S and V' are known,
//   O = diag(γ) Q Sᵀ + M V'.
// Two kernels:
//   prep: W, U, M and K̃ᵀ = (diag(γ_C/γ) K)ᵀ for every (chunk, value head),
//         one workgroup per (chunk, key head) for the Gram tiles the key
//         head's two value heads share;
//   scan: the chunks in order for each (head, 16 value rows), keeping the
//         state slice in LDS, and O for those rows from each chunk's
//         starting S and V' while the next state is being formed.
// Tokens past T in the last chunk enter with k = q = v = 0, β = 0 and
// log g = 0, so they change nothing.
//
// MFMA operand feed: every product is written as D = Σ_k A[i][k] B[j][k] over
// LDS tiles whose rows are k-contiguous. Because the sum is over k, lane
// (r = l % 16, g = l / 16) may hold any k as long as A and B agree: here lane
// group g holds the contiguous k range [g·K/4, (g + 1)·K/4), so each lane
// reads its operands with ds_read_b128, all before the MFMAs. Row strides of
// 4 (mod 64) floats make those reads conflict-free.
#include "conv_common.h"
#include "dh_kernels.h"

namespace dh {

namespace {

constexpr int C = 64;  // tokens per chunk
constexpr int NK = 16, DK = 128, NV = 32, DV = 128;
constexpr int LDF = DK + 4;  // row stride of [.][128] LDS tiles
constexpr int LDT = C + 4;   // row stride of [.][64] LDS tiles
// workspace per (chunk, value head), in floats
constexpr int kOffW = 0;                  // W [64][128]
constexpr int kOffU = kOffW + C * DK;     // U [64][128]
constexpr int kOffM = kOffU + C * DK;     // M [64][64]
constexpr int kOffKt = kOffM + C * C;     // K̃ᵀ [128][64]
constexpr int kOffGam = kOffKt + DK * C;  // γ [64]
constexpr int kWsStride = kOffGam + C;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

__device__ __forceinline__ float softplus_p(float v) { return v > 20.0f ? v : logf(1.0f + expf(v)); }

template <int B, int E, typename Fn>
__device__ __forceinline__ void sfor(Fn&& fn) {
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    sfor<B + 1, E>(fn);
  }
}

// acc += Σ_k A[r][k] B[r][k] over KLEN, A and B pointing at the tiles' first
// rows (16 rows each); lane (r, g) covers k in [g·KLEN/4, (g + 1)·KLEN/4).
template <int KLEN>
__device__ __forceinline__ f4 nt_tile(const float* A, int lda, const float* B, int ldb, int r, int g, f4 acc) {
  constexpr int P = KLEN / 4;
  f4 a[P / 4], b[P / 4];
  const float* pa = A + r * lda + g * P;
  const float* pb = B + r * ldb + g * P;
#pragma unroll
  for (int q = 0; q < P / 4; ++q) {
    a[q] = *(const f4*)(pa + 4 * q);
    b[q] = *(const f4*)(pb + 4 * q);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every read ahead of the MFMAs (the scheduler would interleave them)
  f4 acc2 = f4{0.f, 0.f, 0.f, 0.f};  // two independent chains, summed at the end
#pragma unroll
  for (int q = 0; q < P / 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      acc = mfma4(a[q][e], b[q][e], acc);
      acc2 = mfma4(a[q][e + 1], b[q][e + 1], acc2);
    }
  return acc + acc2;
}

// Rows t0 .. t0 + 63 of a [T][heads][128] fp32 tensor (head `hd`), zero past
// T: thread tid holds float4 number tid + 256 n, row (tid + 256 n) / 32.
__device__ __forceinline__ void fetch_rows(f4 (&x)[8], const float* __restrict__ src, uint32_t t0, uint32_t T,
                                           uint32_t heads, uint32_t hd, int tid) {
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int e = tid + 256 * n, i = e >> 5, d4 = (e & 31) * 4;
    x[n] = t0 + i < T ? *(const f4*)(src + ((size_t)(t0 + i) * heads + hd) * DK + d4) : f4{0.f, 0.f, 0.f, 0.f};
  }
}

__device__ __forceinline__ void stage_rows(float* dst, const f4 (&x)[8], int tid) {
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int e = tid + 256 * n, i = e >> 5, d4 = (e & 31) * 4;
    *(f4*)(dst + i * LDF + d4) = x[n];
  }
}

// The 10 blocks (i, j), j ≤ i, of a 4 × 4 block lower triangle.
__device__ __forceinline__ void lower_block(int p, int& i, int& j) {
  i = p < 1 ? 0 : p < 3 ? 1 : p < 6 ? 2 : 3;
  j = p - i * (i + 1) / 2;
}

}  // namespace

// What prep reads: the conv step's outputs q, k, v, or (fused) the raw
// in-projection p (row stride ldp, the qkv columns first), the conv state
// `prev` [3][CONV_DIM] of the rows before the first and the conv weights, from
// which it forms its own q, k and v (conv_common.h, the stand-alone conv
// kernel's arithmetic) and writes q for the scan to qout.
struct PrepSrc {
  const float* q;
  const float* k;
  const float* v;
  const float* p;
  const float* prev;
  const float* convw;
  float* qout;
  uint32_t ldp;
};

// Where raw conv input row s of channels c, c + 1 (c even) is read from: the conv state for s < 0, else row
// s of p clamped into 0 .. T - 1 (T >= 1), so that the load needs no branch; rows s >= T are zeroed by the
// caller after the load (raw_zero).
__device__ __forceinline__ const f2* raw_ptr(const PrepSrc& in, int s, uint32_t T, uint32_t c) {
  return (const f2*)(s < 0 ? in.prev + (size_t)(3 + s) * convk::CONV_DIM + c
                           : in.p + (size_t)min((uint32_t)s, T - 1) * in.ldp + c);
}
__device__ __forceinline__ f2 raw_zero(f2 x, int s, uint32_t T) { return s < 0 || (uint32_t)s < T ? x : f2{0.f, 0.f}; }

// ---------------------------------------------------------------------------
// prep: one workgroup per (chunk, key head). The Gram tiles Q Kᵀ and K Kᵀ are
// the key head's, shared by its two value heads 2 hk and 2 hk + 1 (which
// differ only in their gates), so they are computed once and scaled for each;
// then waves 4 hh .. 4 hh + 3 do value head 2 hk + hh's inversion, W and U.
// FUSED: the conv step happens here (see PrepSrc), so k and v never go through
// memory and the stand-alone conv kernel does not run.
template <bool FUSED>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(4, 4))) void
delta_chunk_prep_kernel(const PrepSrc src, const float* __restrict__ a,
                                                               const float* __restrict__ b, uint32_t ldab,
                                                               const float* __restrict__ a_log,
                                                               const float* __restrict__ dt_bias, float* __restrict__ ws,
                                                               uint32_t T) {
  // 78 KB of LDS, so that two workgroups of 8 waves fit a CU: Q is staged only for the Gram tiles, whose results
  // wait in registers until every wave is past them; then each value head's A and T take Q's place, sharing one
  // [64][68] tile: A (strictly lower) in the blocks below the diagonal, Tᵀ in the blocks above it, and each
  // diagonal 16 × 16 block holding A_jj until its forward substitution replaces it with the whole T_jjᵀ (A_jj is
  // read by nothing else). V never goes through LDS (each wave loads its U operand into registers during the
  // inversion).
  constexpr int kAT = C * LDT;  // one [64][68] tile
  constexpr int kR2 = C * LDF > 2 * kAT ? C * LDF : 2 * kAT;
  __shared__ __attribute__((aligned(16))) float Ks[C * LDF];
  __shared__ __attribute__((aligned(16))) float R2[kR2];  // Q; then A0 + T0ᵀ | A1 + T1ᵀ
  __shared__ __attribute__((aligned(16))) float Lg[2][C], Bt[2][C], Gm[2][C], SCw[2][C], Rh[2][C];
  __shared__ float Ysc[8 * 16 * 17];  // per-wave 16 × 16 scratch of the blocked inversion
  const uint32_t c = blockIdx.x, hk = blockIdx.y, t0 = c * C;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: per-head values load into SGPRs
  const int r = lane & 15, g = lane >> 4;
  const int hh = wave >> 2, lw = wave & 3;  // this wave's value head (of the key head's two), and its wave in that half
  const uint32_t h = 2 * hk + hh;
  float* const ATs = R2 + hh * kAT;  // A[i][j] at [i][j], T[i][j] at [j][i] (see above)
  float* const out0 = ws + ((size_t)c * NV + 2 * hk) * kWsStride;
  float* const out = out0 + hh * kWsStride;
  // Waves 0 and 4 form value head h's gates after their conv step; their loads go out first, so that the
  // latency overlaps the conv (rows past T read row T - 1 and are dropped below).
  float ga = 0.f, gb = 0.f;
  if (lw == 0) {
    const size_t ta = (size_t)min(t0 + (uint32_t)lane, T - 1) * ldab + h;
    ga = a[ta];
    gb = b[ta];
  }
  // Waves 0 and 4 form value head h's gates after their conv step; their loads go out first, so that the
  // latency overlaps the conv (rows past T read row T - 1 and are dropped below).

  if constexpr (FUSED) {
    // wave w: k (w < 4) or q (w ≥ 4) of key head hk over the chunk's rows 16 (w & 3) .. + 16, lane l owning
    // channels 2l, 2l + 1: the stand-alone conv kernel's (slot, run) unit, evaluated the same way
    const int run = wave & 3;
    const bool isq = wave >= 4;
    const uint32_t c = (uint32_t)(isq ? hk : NK + hk) * DK + 2 * lane;
    const f4 w0 = *(const f4*)(src.convw + (size_t)c * 4), w1 = *(const f4*)(src.convw + (size_t)(c + 1) * 4);
    const int tr0 = (int)t0 + 16 * run;
    f2 x[19];  // raw rows tr0 - 3 .. tr0 + 15, all loads in flight together (no branch between them)
#pragma unroll
    for (int j = 0; j < 19; ++j) x[j] = *raw_ptr(src, tr0 - 3 + j, T, c);
#pragma unroll
    for (int j = 0; j < 19; ++j) x[j] = raw_zero(x[j], tr0 - 3 + j, T);
    float* dst = isq ? R2 : Ks;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const uint32_t t = (uint32_t)(tr0 + u);
      const float y0 = convk::conv_silu(w0, x[u][0], x[u + 1][0], x[u + 2][0], x[u + 3][0]);
      const float y1 = convk::conv_silu(w1, x[u][1], x[u + 1][1], x[u + 2][1], x[u + 3][1]);
      const float inv = convk::l2_inv(y0, y1);
      const float sc = isq ? convk::q_scale(inv) : inv;
      const f2 o = t < T ? f2{y0 * sc, y1 * sc} : f2{0.f, 0.f};
      *(f2*)(dst + (16 * run + u) * LDF + 2 * lane) = o;
      if (isq && t < T) *(f2*)(src.qout + ((size_t)t * NK + hk) * DK + 2 * lane) = o;
    }
  } else {  // threads 0-255 stage K, 256-511 Q; all loads in flight before the first LDS store
    f4 x[8];
    fetch_rows(x, tid < 256 ? src.k : src.q, t0, T, NK, hk, tid & 255);
    stage_rows(tid < 256 ? Ks : R2, x, tid & 255);
  }
  if (lw == 0) {  // waves 0 and 4: value head h's gates
    const uint32_t t = t0 + lane;
    float lam = 0.f, bt = 0.f;
    if (t < T) {
      lam = -expf(a_log[h]) * softplus_p(ga + dt_bias[h]);
      bt = 1.0f / (1.0f + expf(-gb));
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {  // inclusive prefix sum of log g over the chunk
      const float y = __shfl_up(lam, o, 64);
      if (lane >= o) lam += y;
    }
    const float last = __shfl(lam, 63, 64);
    const float gm = expf(lam);
    Lg[hh][lane] = lam;
    Bt[hh][lane] = bt;
    Gm[hh][lane] = gm;
    SCw[hh][lane] = bt * gm;
    Rh[hh][lane] = expf(last - lam);
  }
  __syncthreads();

  // The 20 Gram tiles: tile t < 10 is block t of Q Kᵀ (lower triangle incl. diagonal), t ≥ 10 block t − 10 of
  // K Kᵀ (strictly lower); wave w takes t = w, w + 8, w + 16. Each tile then gives both value heads' M
  // (γ_i/γ_j, to global; the scan reads only the blocks on and below the diagonal) or A (β_i γ_i/γ_j, over Q's
  // LDS). The K rows go in as the MFMA's A operand, so lane (r, g) ends with the tile's row r and columns
  // 4 g .. 4 g + 3 (the same products summed in the same order as with the operands the other way round) and
  // stores them as one 16-byte piece.
  f4 gacc[3];
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int tt = wave + 8 * u;
    if (tt < 20) {
      int ti, tj;
      lower_block(tt < 10 ? tt : tt - 10, ti, tj);
      gacc[u] = nt_tile<DK>(Ks + 16 * tj * LDF, LDF, (tt < 10 ? R2 : Ks) + 16 * ti * LDF, LDF, r, g,
                            f4{0.f, 0.f, 0.f, 0.f});
    }
  }
  __syncthreads();  // every wave is past its Gram tiles: Q is dead
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int tt = wave + 8 * u;
    if (tt < 20) {
      const bool isq = tt < 10;
      int ti, tj;
      lower_block(isq ? tt : tt - 10, ti, tj);
      const int i = 16 * ti + r, j0 = 16 * tj + 4 * g;
#pragma unroll
      for (int vh = 0; vh < 2; ++vh) {
        f4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + e;
          const float rr = i >= j ? expf(Lg[vh][i] - Lg[vh][j]) : 0.f;
          v[e] = isq ? rr * gacc[u][e] : (i > j ? Bt[vh][i] * rr * gacc[u][e] : 0.f);
        }
        if (isq)
          *(f4*)(out0 + vh * kWsStride + kOffM + i * C + j0) = v;
        else
          *(f4*)(R2 + vh * kAT + i * LDT + j0) = v;
      }
    }
  }
  {  // K̃ᵀ[d][j] = (γ_C/γ_j) K[j][d] for the scan; threads 0-255 for value head 2 hk, 256-511 for 2 hk + 1
    const int vh = tid >> 8, t8 = tid & 255;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int e = t8 + 256 * n, d = e >> 4, j4 = (e & 15) * 4;
      f4 x;
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] = Rh[vh][j4 + u] * Ks[(j4 + u) * LDF + d];
      *(f4*)(out0 + vh * kWsStride + kOffKt + d * C + j4) = x;
    }
  }
  if (tid < 2 * C) out0[(tid >> 6) * kWsStride + kOffGam + (tid & 63)] = Gm[tid >> 6][tid & 63];

  // This wave's U operand, V[t0 + 16 jb + 4 g + s][32 lw + 2 r + q2] (its U tile q2 takes the head's value
  // channels 32 lw + 2 ρ + q2, so each lane holds two adjacent channels and loads them as one 8-byte piece),
  // straight into registers; the loads run during the inversion below (fused: its 4 tokens' 7 raw rows per
  // block, conv + SiLU in registers).
  f4 vr[2][4];
  f4 vw[2];       // fused: the conv weights of this lane's two value channels
  f2 vx[4][7];    // fused: raw rows 16 jb + 4 g - 3 .. + 3 of them, combined after the inversion
  const uint32_t cv = 32 * lw + 2 * r;  // this lane's first value channel in the head
  if constexpr (FUSED) {
    const uint32_t c = 2 * convk::KEY_DIM + h * DV + cv;
    vw[0] = *(const f4*)(src.convw + (size_t)c * 4);
    vw[1] = *(const f4*)(src.convw + (size_t)(c + 1) * 4);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int j = 0; j < 7; ++j) vx[jb][j] = *raw_ptr(src, (int)t0 + 16 * jb + 4 * g - 3 + j, T, c);
  } else {
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const uint32_t t = t0 + 16 * jb + 4 * g + s4;
        const f2 x = *(const f2*)(src.v + ((size_t)min(t, T - 1) * NV + h) * DV + cv);  // clamped: no branch
        vr[0][jb][s4] = t < T ? x[0] : 0.f;
        vr[1][jb][s4] = t < T ? x[1] : 0.f;
      }
  }

  // T = (I + A)⁻¹ per value head, blocked 4 × 4 over 16 × 16 blocks. Diagonal blocks by forward
  // substitution (wave lw of the head's half, lane j < 16 owns column j of block lw); then the blocks below
  // the diagonal, one block-diagonal at a time,
  //   T_ij = −T_ii Σ_{k=j}^{i−1} A_ik T_kj,
  // as 16 × 16 MFMA products through a per-wave LDS scratch block.
  __syncthreads();
  {
    const int jb = lw;
    if (lane < 16) {
      float x[16];
      sfor<0, 16>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        float sacc = 0.f;
        sfor<0, i>([&](auto mc) {
          constexpr int m = decltype(mc)::value;
          sacc = fmaf(ATs[(16 * jb + i) * LDT + 16 * jb + m], x[m], sacc);
        });
        x[i] = i == lane ? 1.0f : -sacc;
      });
      sfor<0, 16>([&](auto ic) {  // column lane of T_jj as row lane of T_jjᵀ, over A_jj (every read of it is done)
        constexpr int i = decltype(ic)::value;
        ATs[(16 * jb + lane) * LDT + 16 * jb + i] = x[i];
      });
    }
  }
  __syncthreads();
  for (int d = 1; d < 4; ++d) {
    if (lw < 4 - d) {
      const int j = lw, i = lw + d;
      f4 y = f4{0.f, 0.f, 0.f, 0.f};
      for (int kb = j; kb < i; ++kb) {  // Y = Σ_k A_ik T_kj
#pragma unroll
        for (int kk = 0; kk < 16; kk += 4)  // A[16 i + r][16 kb + kk + g] T[16 kb + kk + g][16 j + r]
          y = mfma4(ATs[(16 * i + r) * LDT + 16 * kb + kk + g], ATs[(16 * j + r) * LDT + 16 * kb + kk + g], y);
      }
      float* Yw = Ysc + wave * 16 * 17;
#pragma unroll
      for (int e = 0; e < 4; ++e) Yw[(4 * g + e) * 17 + r] = y[e];
      __builtin_amdgcn_wave_barrier();
      f4 z = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 16; kk += 4)  // T[16 i + r][16 i + kk + g]
        z = mfma4(ATs[(16 * i + kk + g) * LDT + 16 * i + r], Yw[(kk + g) * 17 + r], z);
#pragma unroll
      for (int e = 0; e < 4; ++e) ATs[(16 * j + r) * LDT + 16 * i + 4 * g + e] = -z[e];
    }
    __syncthreads();
  }

  if constexpr (FUSED) {
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          // raw rows past T enter only outputs of tokens past T, which are zero
          const f2* x = vx[jb];
          vr[q2][jb][s4] = t0 + 16 * jb + 4 * g + s4 < T
                               ? convk::conv_silu(vw[q2], x[s4][q2], x[s4 + 1][q2], x[s4 + 2][q2], x[s4 + 3][q2])
                               : 0.f;
        }
  }

  // W = T diag(βγ) K and U = T diag(β) V. Wave lw of the head's half: key/value channels 32 lw .. + 32, as two
  // 16-channel tiles q2 (W: channels 32 lw + 16 q2 + ρ; U: 32 lw + 2 ρ + q2, the order its operand was loaded
  // in). T is lower triangular, so row block ti sums over token blocks jb ≤ ti; within a block lane group g
  // holds tokens 16 jb + 4 g .. + 4 (one ds_read_b128 of the scale; K[j][32 lw + 16 q2 + r] is conflict-free
  // with the row stride of 132 floats, V's comes from registers). The channels go in as the MFMA's A operand,
  // so lane (r, g) ends with token row 16 ti + r and 4 channels of each tile (the same products summed in the
  // same order as with the operands the other way round), which it stores as 16-byte pieces: W's 4 adjacent
  // channels per tile, and U's 8 adjacent channels of both tiles, interleaved.
#pragma unroll
  for (int isu = 0; isu < 2; ++isu) {
    const float* sc = isu ? Bt[hh] : SCw[hh];
    float* dst = out + (isu ? kOffU : kOffW);
    sfor<0, 4>([&](auto tic) {
      constexpr int ti = decltype(tic)::value;
      f4 tv[ti + 1];  // T[16 ti + r][16 jb + 4 g + s] · scale
#pragma unroll
      for (int jb = 0; jb <= ti; ++jb) {
        const f4 sv = *(const f4*)(sc + 16 * jb + 4 * g);
#pragma unroll
        for (int s = 0; s < 4; ++s) tv[jb][s] = ATs[(16 * jb + 4 * g + s) * LDT + 16 * ti + r] * sv[s];
      }
      f4 acc[2];
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        f4 rb[ti + 1];
#pragma unroll
        for (int jb = 0; jb <= ti; ++jb) {
          if (isu) {
            rb[jb] = vr[q2][jb];
          } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) rb[jb][s] = Ks[(16 * jb + 4 * g + s) * LDF + 32 * lw + 16 * q2 + r];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        acc[q2] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jb = 0; jb <= ti; ++jb)
#pragma unroll
          for (int s = 0; s < 4; ++s) acc[q2] = mfma4(rb[jb][s], tv[jb][s], acc[q2]);
      }
      float* row = dst + (16 * ti + r) * DK + 32 * lw;
      if (isu) {
        *(f4*)(row + 8 * g) = f4{acc[0][0], acc[1][0], acc[0][1], acc[1][1]};
        *(f4*)(row + 8 * g + 4) = f4{acc[0][2], acc[1][2], acc[0][3], acc[1][3]};
      } else {
        *(f4*)(row + 4 * g) = acc[0];
        *(f4*)(row + 16 + 4 * g) = acc[1];
      }
    });
  }
}

// ---------------------------------------------------------------------------
// scan: one workgroup per (value head, 16 value rows); the 8 workgroups of a
// head have ids 32 apart, so they run on one XCD and share its L2 for the
// per-chunk matrices. Waves 0-3 carry the recurrence and touch global memory
// only to DMA the next chunk's tiles where they would otherwise wait at a
// barrier; waves 4-7 ("out waves", one per 16 tokens of the chunk) form the
// chunk's output:
//   chunk c, waves 0-3:  V'ᵀ = Uᵀ − S Wᵀ (wave w: tokens 16 w .. + 16); DMA
//                        a quarter of chunk c + 1's W and U slice into the
//                        other LDS buffer
//                        | barrier |
//                        S = γ_C S + V'ᵀ K̃ (wave w: key columns 32 w .. + 32);
//                        DMA a quarter of chunk c + 1's K̃ᵀ; wait for the W
//                        and U DMAs
//   chunk c, waves 4-7:  X = Q Sᵀ for their tokens (S is still the chunk's
//                        starting state), loading chunk c + 1's Q rows
//                        between the products
//                        | barrier |
//                        O = diag(γ) X + M V' (V' complete), loading chunk
//                        c + 1's M rows and γ first; stored
//   | barrier |
// W and K̃ᵀ land by global→LDS DMA (16 bytes per lane, 1 KB per instruction)
// in an unpadded layout whose 16-byte chunks are XOR-swizzled by row
// (chunk c of row r at c ^ (r % 16)), so the MFMA operand reads stay
// conflict-free. An out wave's Q and M rows go straight into registers, in
// the MFMA's k layout, one chunk ahead.
constexpr int kScanRows = 16;

// Wave-uniform copies in SGPRs (the DMA below takes its LDS address and its
// base as scalar operands).
__device__ __forceinline__ uint32_t sgpr_u32(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t sgpr_ptr(const void* p) {
  const uint64_t b = (uint64_t)(uintptr_t)p;
  return ((uint64_t)sgpr_u32((uint32_t)(b >> 32)) << 32) | sgpr_u32((uint32_t)b);
}

// 16 bytes per lane global → LDS: lane l's 16 bytes at sbase + voff land at
// LDS byte address lds_byte + 16·l. M0 is written in the same statement (one
// wait state before its use); nothing else in this file reads M0. Callers
// pass SGPR values made once per batch with sgpr_u32 / sgpr_ptr (and SALU
// offsets from them). A VMEM instruction may read an SGPR only 5 wait states
// after a VALU instruction (readfirstlane) wrote it, and the compiler, which
// places the readfirstlane, cannot see the load inside the asm string: the
// first DMA of a batch (PAD) supplies them itself with s_nop 4, the rest of
// the batch reads SGPRs written long before. The build checks the generated
// code for that (check_dma_hazard.py).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool PAD = false>
__device__ __forceinline__ void dma16_lds(uint32_t lds_byte, uint32_t voff, uint64_t sbase) {
  if constexpr (PAD)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %1, %2 offset:0" ::"s"(lds_byte), "v"(voff),
                 "s"((const void*)(uintptr_t)sbase)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:0" ::"s"(lds_byte), "v"(voff),
                 "s"((const void*)(uintptr_t)sbase)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// acc += Σ_k A[r][k] B[r][k] with A a padded LDS tile (row stride lda floats)
// and B an XOR-swizzled tile of CH 16-byte chunks per row starting at row b0
// (b0 % 16 == 0); lane (r, g) covers k in [g·KLEN/4, (g + 1)·KLEN/4).
template <int KLEN, int CH>
__device__ __forceinline__ f4 nt_tile_swz(const float* A, int lda, const float* B, int b0, int r, int g, f4 acc) {
  constexpr int P = KLEN / 4, Q = P / 4;
  f4 a[Q], b[Q];
  const float* pa = A + r * lda + g * P;
  const float* pb = B + (b0 + r) * CH * 4;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    a[q] = *(const f4*)(pa + 4 * q);
    b[q] = *(const f4*)(pb + 4 * ((g * Q + q) ^ r));
  }
  __builtin_amdgcn_sched_barrier(0);
  f4 acc2 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      acc = mfma4(a[q][e], b[q][e], acc);
      acc2 = mfma4(a[q][e + 1], b[q][e + 1], acc2);
    }
  return acc + acc2;
}

// Two tiles that share A: acc0 += Σ_k A[r][k] B[b0 + r][k] and acc1 the same
// with rows b1 of B, in nt_tile_swz's order per tile (two chains each, summed
// at the end) but with one read of A and the four chains interleaved.
template <int KLEN, int CH>
__device__ __forceinline__ void nt_tile2_swz(const float* A, int lda, const float* B, int b0, int b1, int r, int g,
                                             f4& acc0, f4& acc1) {
  constexpr int P = KLEN / 4, Q = P / 4;
  f4 a[Q], u[Q], w[Q];
  const float* pa = A + r * lda + g * P;
  const float* pu = B + (b0 + r) * CH * 4;
  const float* pw = B + (b1 + r) * CH * 4;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    a[q] = *(const f4*)(pa + 4 * q);
    u[q] = *(const f4*)(pu + 4 * ((g * Q + q) ^ r));
    w[q] = *(const f4*)(pw + 4 * ((g * Q + q) ^ r));
  }
  __builtin_amdgcn_sched_barrier(0);
  f4 acc0b = f4{0.f, 0.f, 0.f, 0.f}, acc1b = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      acc0 = mfma4(a[q][e], u[q][e], acc0);
      acc1 = mfma4(a[q][e], w[q][e], acc1);
      acc0b = mfma4(a[q][e + 1], u[q][e + 1], acc0b);
      acc1b = mfma4(a[q][e + 1], w[q][e + 1], acc1b);
    }
  acc0 += acc0b;
  acc1 += acc1b;
}

__global__ __launch_bounds__(512) void delta_chunk_scan_kernel(float* __restrict__ ws, const float* __restrict__ q,
                                                               const float* state_in, float* state_out,
                                                               float* __restrict__ o, uint32_t T,
                                                               uint32_t write_state) {
  __shared__ __attribute__((aligned(16))) float Ss[kScanRows * LDF];
  __shared__ __attribute__((aligned(1024))) float Wb[2][C * DK];   // [64 tokens][32 chunks], swizzled
  __shared__ __attribute__((aligned(1024))) float Kb[2][DK * C];   // [128 keys][16 chunks], swizzled
  __shared__ __attribute__((aligned(1024))) float Ub[2][C * kScanRows];  // [64 tokens][16 values]
  __shared__ __attribute__((aligned(16))) float Vt[kScanRows * LDT];
  __shared__ float Gc[2];
  const uint32_t h = blockIdx.x, hk = h >> 1, dv0 = blockIdx.y * kScanRows;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // in an SGPR: the DMA's LDS offsets derive from it
  const int r = lane & 15, g = lane >> 4;
  const uint32_t nch = (T + C - 1) / C;
  auto slot = [&](uint32_t c) { return ws + ((size_t)c * NV + h) * kWsStride; };

  // The next chunk's operands are loaded during this one: W, K̃ᵀ and the U slice by DMA into buffer bf ^ 1, each
  // recurrence wave its quarter, issued where that wave would otherwise wait at a barrier (W and U after its V'
  // products, K̃ᵀ after its state update: each has the following phase to land); Q, M and γ rows into the out
  // waves' registers, spread over their products. The vector memory unit passes about one 1 KB instruction per
  // 30 clocks for the whole CU, and a wave stalls at each instruction it cannot hand over: issued back to back
  // by the out waves, the chunk's 114 instructions held them (and through the barriers, the recurrence) for
  // most of each phase.
  struct DmaBase {
    uint64_t bw, bk, bu;
    uint32_t wl, kl, ul;
  };
  auto dma_base = [&](uint32_t c, int bf) {
    const float* in = slot(c);
    DmaBase d;
    d.bw = sgpr_ptr(in + kOffW);
    d.bk = sgpr_ptr(in + kOffKt);
    d.bu = sgpr_ptr(in + kOffU);
    d.wl = sgpr_u32((uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)Wb[bf]);
    d.kl = sgpr_u32((uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)Kb[bf]);
    d.ul = sgpr_u32((uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)Ub[bf]);
    return d;
  };
  const int qw = wave & 3, n0 = 8 * qw;  // a recurrence wave's quarter of the DMA'd tiles
  // W: LDS chunk 64 n + lane = row 2 n + lane / 32, slot lane % 32
  auto dma_w = [&](int n) {
    const int row = 2 * n + (lane >> 5), c4 = (lane & 31) ^ (row & 15);
    return (uint32_t)((row * DK + 4 * c4) * 4);
  };
  // K̃ᵀ: row 4 n + lane / 16, slot lane % 16
  auto dma_k = [&](int n) {
    const int row = 4 * n + (lane >> 4), c4 = (lane & 15) ^ (row & 15);
    return (uint32_t)((row * C + 4 * c4) * 4);
  };
  // U rows, columns dv0 .. + 16: row 16 qw + lane / 4, chunk lane % 4
  const uint32_t u_off = (uint32_t)(((16 * qw + (lane >> 2)) * DK + dv0 + 4 * (lane & 3)) * 4);
  // The 8 workgroups of a head read the same tiles at about the same time; each starts its 8 contiguous 1 KB
  // pieces at a different one (rotation by its value-row slice), so that they do not all queue on the same lines.
  const int rot = (int)blockIdx.y & 7;
  auto dma_wu = [&](const DmaBase& d) {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int p = n0 + ((n + rot) & 7);
      if (n == 0)
        dma16_lds<true>(d.wl + p * 1024, dma_w(p), d.bw);
      else
        dma16_lds(d.wl + p * 1024, dma_w(p), d.bw);
    }
    dma16_lds(d.ul + qw * 1024, u_off, d.bu);
  };
  auto dma_kt = [&](const DmaBase& d) {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int p = n0 + ((n + rot) & 7);
      if (n == 0)
        dma16_lds<true>(d.kl + p * 1024, dma_k(p), d.bk);
      else
        dma16_lds(d.kl + p * 1024, dma_k(p), d.bk);
    }
  };
  // an out wave's operands for chunk c: Q[t0 + i0 + r][16 n + 4 g .. + 4] (n < 8: each load instruction reads
  // 64 contiguous bytes per row, four lanes to a row, where a 32-float run per lane made every lane's 16 bytes a
  // cache line of its own), M[i0 + r][16 jb + 4 g .. + 4] (jb ≤ ow), and γ of the tokens its output lanes hold
  const int ow = wave - 4, i0 = 16 * ow;
  f4 qa[8], ma[4], gi;  // this chunk's
  f4 qn[8], mn[4], gn;  // the next chunk's, loaded during this one
  auto load_q = [&](uint32_t c, int n) {
    const uint32_t t = c * C + i0 + r;
    const float* qr = q + ((size_t)min(t, T - 1) * NK + hk) * DK + 4 * g;  // rows past T: any finite row
    qn[n] = *(const f4*)(qr + 16 * n);
  };
  auto load_mg = [&](uint32_t c) {
    gn = *(const f4*)(slot(c) + kOffGam + i0 + 4 * g);
    const float* mr = slot(c) + kOffM + (i0 + r) * C + 4 * g;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) mn[jb] = jb <= ow ? *(const f4*)(mr + 16 * jb) : f4{0.f, 0.f, 0.f, 0.f};
  };
  // The copies happen here, not where the compiler would sink them (the loop's latch, behind the output stores,
  // with a full wait on them): the empty asm makes each copy's result a value defined at this point.
  auto take_ops = [&]() {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      qa[n] = qn[n];
      asm volatile("" : "+v"(qa[n]));
    }
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      ma[jb] = mn[jb];
      asm volatile("" : "+v"(ma[jb]));
    }
    gi = gn;
    asm volatile("" : "+v"(gi));
  };

  if (wave >= 4) {
#pragma unroll
    for (int n = 0; n < 8; ++n) load_q(0, n);
    load_mg(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    take_ops();
    if (wave == 7 && lane == 48) Gc[0] = gi[3];  // γ of the chunk's last token
  } else {
    const DmaBase d = dma_base(0, 0);
    dma_wu(d);
    dma_kt(d);
    for (int e = tid; e < kScanRows * DK / 4; e += 256) {
      const int row = e >> 5, d4 = (e & 31) * 4;
      *(f4*)(Ss + row * LDF + d4) = *(const f4*)(state_in + ((size_t)h * DV + dv0 + row) * DK + d4);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // the recurrence's waves issue first when both waves of a SIMD are ready: the out waves fill the gaps
    __builtin_amdgcn_s_setprio(3);
  }
  __syncthreads();

  for (uint32_t c = 0; c < nch; ++c) {
    const int bf = c & 1;
    const bool more = c + 1 < nch;
    f4 x;
    DmaBase dn;
    if (wave >= 4) {
      // X[i][dv] = Σ_d Q[i][d] S[dv][d] with S the chunk's starting state, the next Q rows loaded between
      f4 sb[8];
      const float* sr = Ss + r * LDF + 4 * g;
#pragma unroll
      for (int n = 0; n < 8; ++n) sb[n] = *(const f4*)(sr + 16 * n);
      __builtin_amdgcn_sched_barrier(0);
      f4 x2 = f4{0.f, 0.f, 0.f, 0.f};
      x = f4{0.f, 0.f, 0.f, 0.f};
      sfor<0, 16>([&](auto ic) {
        constexpr int it = decltype(ic)::value, n = it / 2, e = 2 * (it % 2);
        if constexpr (e == 0) {
          if (more) load_q(c + 1, n);
        }
        x = mfma4(qa[n][e], sb[n][e], x);
        x2 = mfma4(qa[n][e + 1], sb[n][e + 1], x2);
        __builtin_amdgcn_sched_barrier(0);
      });
      x = (x + x2) * gi;
    } else {  // V'ᵀ[dv][i] = U[i][dv] − Σ_d S[dv][d] W[i][d]
      if (more) dn = dma_base(c + 1, bf ^ 1);  // buffers bf ^ 1 were last read during chunk c - 1
      const int iw = 16 * wave;
      const f4 acc = nt_tile_swz<DK, 32>(Ss, LDF, Wb[bf], iw, r, g, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int dv = 4 * g + e, i = iw + r;
        Vt[dv * LDT + i] = Ub[bf][i * kScanRows + dv] - acc[e];
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of K̃ᵀ for this chunk (a phase ago)
      if (more) dma_wu(dn);
    }
    __syncthreads();  // V'ᵀ complete; every read of S for V' and X done; K̃ᵀ in place
    if (wave >= 4) {  // O[i][dv] = γ_i X[i][dv] + Σ_{j ≤ i} M[i][j] V'ᵀ[dv][j]
      if (more) load_mg(c + 1);
      f4 vb[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) vb[jb] = *(const f4*)(Vt + r * LDT + 16 * jb + 4 * g);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        if (jb <= ow) {
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) x = mfma4(ma[jb][s4], vb[jb][s4], x);
        }
      }
      // the next chunk's rows have landed; they move into place before the stores go out, so that no wait the
      // compiler places for those registers (a full one, with stores in flight) falls behind the stores
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      take_ops();
      if (wave == 7 && lane == 48 && more) Gc[bf ^ 1] = gi[3];  // γ of the next chunk's last token
      const uint32_t tb = c * C + i0 + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (tb + e < T) o[((size_t)(tb + e) * NV + h) * DV + dv0 + r] = x[e];
    } else {  // S[dv][d] ← γ_C S[dv][d] + Σ_j V'ᵀ[dv][j] K̃ᵀ[d][j]; each wave reads and writes only its own columns
      const float gC = Gc[bf];
      const int d0 = 32 * wave;
      f4 acc0, acc1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc0[e] = gC * Ss[(4 * g + e) * LDF + d0 + r];
        acc1[e] = gC * Ss[(4 * g + e) * LDF + d0 + 16 + r];
      }
      nt_tile2_swz<C, 16>(Vt, LDT, Kb[bf], d0, d0 + 16, r, g, acc0, acc1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Ss[(4 * g + e) * LDF + d0 + r] = acc0[e];
        Ss[(4 * g + e) * LDF + d0 + 16 + r] = acc1[e];
      }
      if (more) {
        dma_kt(dn);
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // this wave's W and U for the next chunk; K̃ᵀ in flight
      }
    }
    __syncthreads();  // S and the next chunk's tiles are in place
  }
  if (write_state && wave < 4) {
    for (int e = tid; e < kScanRows * DK / 4; e += 256) {
      const int row = e >> 5, d4 = (e & 31) * 4;
      *(f4*)(state_out + ((size_t)h * DV + dv0 + row) * DK + d4) = *(const f4*)(Ss + row * LDF + d4);
    }
  }
}

size_t delta_chunk_ws_floats(uint32_t t) { return (size_t)((t + C - 1) / C) * NV * kWsStride; }

hipError_t launch_gated_delta_chunked(const float* q, const float* k, const float* v, const float* a, const float* b,
                                      const float* a_log, const float* dt_bias, const float* state_in,
                                      float* state_out, float* o, float* ws, uint32_t t, uint32_t ldab,
                                      bool write_state, hipStream_t s) {
  const uint32_t nch = (t + C - 1) / C;
  const PrepSrc src{q, k, v, nullptr, nullptr, nullptr, nullptr, 0};
  hipLaunchKernelGGL(delta_chunk_prep_kernel<false>, dim3(nch, NK), dim3(512), 0, s, src, a, b, ldab, a_log, dt_bias,
                     ws, t);
  hipLaunchKernelGGL(delta_chunk_scan_kernel, dim3(NV, DV / kScanRows), dim3(512), 0, s, ws, q, state_in, state_out, o,
                     t, write_state ? 1u : 0u);
  return hipGetLastError();
}

hipError_t launch_conv_gated_delta_chunked(const float* p, const float* prev, const float* conv_w, uint32_t ldp,
                                           float* q, const float* a, const float* b, uint32_t ldab,
                                           const float* a_log, const float* dt_bias, const float* state_in,
                                           float* state_out, float* o, float* ws, uint32_t t, bool write_state,
                                           hipStream_t s) {
  const uint32_t nch = (t + C - 1) / C;
  const PrepSrc src{nullptr, nullptr, nullptr, p, prev, conv_w, q, ldp};
  hipLaunchKernelGGL(delta_chunk_prep_kernel<true>, dim3(nch, NK), dim3(512), 0, s, src, a, b, ldab, a_log, dt_bias,
                     ws, t);
  hipLaunchKernelGGL(delta_chunk_scan_kernel, dim3(NV, DV / kScanRows), dim3(512), 0, s, ws, q, state_in, state_out, o,
                     t, write_state ? 1u : 0u);
  return hipGetLastError();
}

}  // namespace dh
