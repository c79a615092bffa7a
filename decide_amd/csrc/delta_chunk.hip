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
// then, sequentially over chunks with the state S (DV × DK) of the chunk start,
//   V' = U − W Sᵀ,   O = diag(γ) Q Sᵀ + M V',   S ← γ_C S + V'ᵀ diag(γ_C/γ) K.
// Kernel 1 (prep) computes A, T, W, U, M for every (chunk, value head) in
// parallel; kernel 2 (scan) runs the chunks in order for each (head, 32 value
// rows). Tokens past T in the last chunk enter with k = q = v = 0, β = 0 and
// log g = 0, so they change nothing.
#include <type_traits>

#include "dh_kernels.h"

namespace dh {

namespace {

constexpr int C = 64;            // tokens per chunk
constexpr int NK = 16, DK = 128, NV = 32, DV = 128;
// LDS row strides, in floats, for 64 banks of 4 bytes. A tile read as an
// MFMA operand with lane (r, g) at [16 m + r][4 n + g] needs a stride of 4
// (mod 64) to be conflict-free; one read at [4 n + g][16 m + r] (the B
// operand of a product over the tile's rows) needs 16 (mod 64).
constexpr int LDF = DK + 4;      // 64 × 128 tiles read along rows
constexpr int LDK = DK + 16;     // 64 × 128 tiles read down columns
constexpr int LDT = C + 4;       // 64 × 64 triangular tiles
constexpr int LDM = C + 4;
// workspace layout per (chunk, value head), in floats
constexpr int kOffW = 0, kOffU = C * DK, kOffM = 2 * C * DK, kOffGam = 2 * C * DK + C * C, kOffRho = kOffGam + C;
constexpr int kWsStride = kOffRho + C;

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

__device__ __forceinline__ float softplus_p(float v) { return v > 20.0f ? v : logf(1.0f + expf(v)); }

template <int B, int E, typename Fn>
__device__ __forceinline__ void sfor(Fn&& fn) {
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    sfor<B + 1, E>(fn);
  }
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

template <int LD>
__device__ __forceinline__ void stage_rows(float* dst, const f4 (&x)[8], int tid) {
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int e = tid + 256 * n, i = e >> 5, d4 = (e & 31) * 4;
    *(f4*)(dst + i * LD + d4) = x[n];
  }
}

// The 10 blocks (i, j), j ≤ i, of a 4 × 4 block lower triangle.
__device__ __forceinline__ void lower_block(int p, int& i, int& j) {
  i = p < 1 ? 0 : p < 3 ? 1 : p < 6 ? 2 : 3;
  j = p - i * (i + 1) / 2;
}

}  // namespace

__global__ __launch_bounds__(256) void delta_chunk_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                               const float* __restrict__ v, const float* __restrict__ a,
                                                               const float* __restrict__ b, uint32_t ldab,
                                                               const float* __restrict__ a_log,
                                                               const float* __restrict__ dt_bias, float* __restrict__ ws,
                                                               uint32_t T) {
  __shared__ __attribute__((aligned(16))) float Ks[C * LDF];
  __shared__ __attribute__((aligned(16))) float Qs[C * LDF];
  __shared__ __attribute__((aligned(16))) float Vs[C * LDK];
  __shared__ float As[C * LDT];
  __shared__ float Ts[C * LDT];
  __shared__ float Lg[C], Bt[C], Gm[C];
  __shared__ float Ysc[4 * 16 * 17];  // per-wave 16 × 16 scratch of the blocked inversion
  const uint32_t c = blockIdx.x, h = blockIdx.y, hk = h >> 1, t0 = c * C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  float* out = ws + ((size_t)c * NV + h) * kWsStride;

  {  // all 24 loads in flight before the first LDS store
    f4 xk[8], xq[8], xv[8];
    fetch_rows(xk, k, t0, T, NK, hk, tid);
    fetch_rows(xq, q, t0, T, NK, hk, tid);
    fetch_rows(xv, v, t0, T, NV, h, tid);
    stage_rows<LDF>(Ks, xk, tid);
    stage_rows<LDF>(Qs, xq, tid);
    stage_rows<LDK>(Vs, xv, tid);
  }
  if (wave == 0) {
    const uint32_t t = t0 + lane;
    float lam = 0.f, bt = 0.f;
    if (t < T) {
      lam = -expf(a_log[h]) * softplus_p(a[(size_t)t * ldab + h] + dt_bias[h]);
      bt = 1.0f / (1.0f + expf(-b[(size_t)t * ldab + h]));
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {  // inclusive prefix sum of log g over the chunk
      const float y = __shfl_up(lam, o, 64);
      if (lane >= o) lam += y;
    }
    Lg[lane] = lam;
    Bt[lane] = bt;
    Gm[lane] = expf(lam);
  }
  __syncthreads();

  // K Kᵀ → A (strictly lower, β_i γ_i/γ_j), Q Kᵀ → M (lower incl. diagonal, γ_i/γ_j): the 2 × 10 blocks
  // of 16 × 16 on or below the diagonal; M's blocks above it are written as zeros, A's are never read
  for (int tt = wave; tt < 20; tt += 4) {
    const bool isq = tt >= 10;
    int ti, tj;
    lower_block(isq ? tt - 10 : tt, ti, tj);
    const float* L = isq ? Qs : Ks;
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int kk = 0; kk < DK; kk += 4)
      acc = mfma4(L[(16 * ti + r16) * LDF + kk + g4], Ks[(16 * tj + r16) * LDF + kk + g4], acc);
    const int j = 16 * tj + r16;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * ti + 4 * g4 + e;
      const float r = i >= j ? expf(Lg[i] - Lg[j]) : 0.f;
      if (!isq)
        As[i * LDT + j] = i > j ? Bt[i] * r * acc[e] : 0.f;
      else
        out[kOffM + i * C + j] = r * acc[e];
    }
  }
  for (int e = tid; e < C * C; e += 256)
    if ((e & 63) >> 4 > e >> 10) out[kOffM + e] = 0.f;
  __syncthreads();

  // T = (I + A)⁻¹, blocked 4 × 4 over 16 × 16 blocks. Diagonal blocks by forward
  // substitution (wave w, lane j < 16 owns column j of block w); then the
  // blocks below the diagonal, one block-diagonal at a time,
  //   T_ij = −T_ii Σ_{k=j}^{i−1} A_ik T_kj,
  // as 16 × 16 MFMA products through a per-wave LDS scratch block.
  for (int e = tid; e < C * LDT; e += 256) Ts[e] = 0.f;
  __syncthreads();
  {
    const int jb = wave;  // diagonal block
    if (lane < 16) {
      float x[16];
      sfor<0, 16>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        float sacc = 0.f;
        sfor<0, i>([&](auto mc) {
          constexpr int m = decltype(mc)::value;
          sacc = fmaf(As[(16 * jb + i) * LDT + 16 * jb + m], x[m], sacc);
        });
        x[i] = i == lane ? 1.0f : -sacc;
      });
      sfor<0, 16>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        Ts[(16 * jb + i) * LDT + 16 * jb + lane] = x[i];
      });
    }
  }
  __syncthreads();
  for (int d = 1; d < 4; ++d) {
    if (wave < 4 - d) {
      const int j = wave, i = wave + d;
      f4 y = f4{0.f, 0.f, 0.f, 0.f};
      for (int kb = j; kb < i; ++kb) {  // Y = Σ_k A_ik T_kj
#pragma unroll
        for (int kk = 0; kk < 16; kk += 4)
          y = mfma4(As[(16 * i + r16) * LDT + 16 * kb + kk + g4], Ts[(16 * kb + kk + g4) * LDT + 16 * j + r16], y);
      }
      float* Yw = Ysc + wave * 16 * 17;
#pragma unroll
      for (int e = 0; e < 4; ++e) Yw[(4 * g4 + e) * 17 + r16] = y[e];
      __builtin_amdgcn_wave_barrier();
      f4 z = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 16; kk += 4)
        z = mfma4(Ts[(16 * i + r16) * LDT + 16 * i + kk + g4], Yw[(kk + g4) * 17 + r16], z);
#pragma unroll
      for (int e = 0; e < 4; ++e) Ts[(16 * i + 4 * g4 + e) * LDT + 16 * j + r16] = -z[e];
    }
    __syncthreads();
  }

  // W = T diag(βγ) K and U = T diag(β) V: 2 × 32 tiles of 16 × 16; T is lower triangular, so row block
  // ti sums over tokens j < 16 (ti + 1) only
  for (int tt = wave; tt < 64; tt += 4) {
    const bool isu = tt >= 32;
    const int ti = (tt & 31) >> 3, td = tt & 7;
    const float* R = isu ? Vs : Ks;
    const int ld = isu ? LDK : LDF;
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
    for (int jj = 0; jj < 16 * (ti + 1); jj += 4) {
      const int j = jj + g4;
      const float sc = isu ? Bt[j] : Bt[j] * Gm[j];
      acc = mfma4(Ts[(16 * ti + r16) * LDT + j], R[j * ld + 16 * td + r16] * sc, acc);
    }
    float* dst = out + (isu ? kOffU : kOffW);
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[(16 * ti + 4 * g4 + e) * DK + 16 * td + r16] = acc[e];
  }
  if (tid < C) {
    out[kOffGam + tid] = Gm[tid];
    out[kOffRho + tid] = expf(Lg[C - 1] - Lg[tid]);
  }
}

// One workgroup of 8 waves per (value head, 32 value rows): the 4 workgroups
// of a head land on one XCD (their ids are 32 apart), so the per-chunk
// matrices they all read come from HBM once and from that XCD's L2 after.
// The state slice S [32][128] stays in LDS across all chunks; the next
// chunk's matrices are loaded into registers while the current chunk
// computes. Wave w owns value tile u = w % 2 and token tile w / 2 of V' and
// O, and key-dim tiles 2 (w / 2), 2 (w / 2) + 1 of the state update.
constexpr int kScanRows = 32, kScanThreads = 512;
constexpr int LDV2 = 48;  // V'ᵀ/U tiles [64][32], read down columns

namespace {
struct ScanPrefetch {
  f4 w[4], q[4], k[4], m[2], u;
  float gam, rho;
};
}  // namespace

__global__ __launch_bounds__(kScanThreads) void delta_chunk_scan_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ ws, const float* state_in,
    float* state_out, float* __restrict__ o, uint32_t T, uint32_t write_state) {
  __shared__ __attribute__((aligned(16))) float Ss[kScanRows * LDF];
  __shared__ __attribute__((aligned(16))) float Ws[C * LDF];
  __shared__ __attribute__((aligned(16))) float Qs[C * LDF];
  __shared__ __attribute__((aligned(16))) float Ks[C * LDK];
  __shared__ float Ms[C * LDM];
  __shared__ float Us[C * LDV2];
  __shared__ float Vp[C * LDV2];
  __shared__ float Gm[C], Rh[C];
  const uint32_t h = blockIdx.x, hk = h >> 1, dv0 = blockIdx.y * kScanRows;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int u = wave & 1, i0 = 16 * (wave >> 1);

  for (int e = tid; e < kScanRows * DK / 4; e += kScanThreads) {
    const int r = e >> 5, d4 = (e & 31) * 4;
    *(f4*)(Ss + r * LDF + d4) = *(const f4*)(state_in + ((size_t)h * DV + dv0 + r) * DK + d4);
  }
  // thread tid moves float4 number e = tid + 512 n of each 64 × 128 tile: row e / 32, columns 4 (e % 32)
  auto fetch = [&](uint32_t c, ScanPrefetch& pf) {
    const float* in = ws + ((size_t)c * NV + h) * kWsStride;
    const uint32_t t0 = c * C;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int e = tid + kScanThreads * n, i = e >> 5, d4 = (e & 31) * 4;
      pf.w[n] = *(const f4*)(in + kOffW + i * DK + d4);
      const uint32_t t = min(t0 + i, T - 1);  // rows past T: any finite row (their W, U, M rows are 0)
      pf.q[n] = *(const f4*)(q + ((size_t)t * NK + hk) * DK + d4);
      pf.k[n] = t0 + i < T ? *(const f4*)(k + ((size_t)t * NK + hk) * DK + d4) : f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int n = 0; n < 2; ++n) pf.m[n] = *(const f4*)(in + kOffM + (tid + kScanThreads * n) * 4);
    pf.u = *(const f4*)(in + kOffU + (tid >> 3) * DK + dv0 + (tid & 7) * 4);
    pf.gam = tid < C ? in[kOffGam + tid] : 0.f;
    pf.rho = tid < C ? in[kOffRho + tid] : 0.f;
  };
  auto stage = [&](const ScanPrefetch& pf) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int e = tid + kScanThreads * n, i = e >> 5, d4 = (e & 31) * 4;
      *(f4*)(Ws + i * LDF + d4) = pf.w[n];
      *(f4*)(Qs + i * LDF + d4) = pf.q[n];
      *(f4*)(Ks + i * LDK + d4) = pf.k[n];
    }
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int e = (tid + kScanThreads * n) * 4, i = e >> 6, j = e & 63;
      *(f4*)(Ms + i * LDM + j) = pf.m[n];
    }
    *(f4*)(Us + (tid >> 3) * LDV2 + (tid & 7) * 4) = pf.u;
    if (tid < C) {
      Gm[tid] = pf.gam;
      Rh[tid] = pf.rho;
    }
  };

  const uint32_t nch = (T + C - 1) / C;
  ScanPrefetch pf;
  fetch(0, pf);
  for (uint32_t c = 0; c < nch; ++c) {
    const uint32_t t0 = c * C;
    __syncthreads();  // the previous chunk's reads of the staged tiles are done
    stage(pf);
    __syncthreads();
    if (c + 1 < nch) fetch(c + 1, pf);  // in flight while this chunk computes

    // V'ᵀ[dv][i] = Uᵀ − S Wᵀ on (value tile u, token tile i0)
    {
      f4 a0 = f4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll 8
      for (int kk = 0; kk < DK; kk += 8) {
        a0 = mfma4(Ss[(16 * u + r16) * LDF + kk + g4], Ws[(i0 + r16) * LDF + kk + g4], a0);
        a1 = mfma4(Ss[(16 * u + r16) * LDF + kk + 4 + g4], Ws[(i0 + r16) * LDF + kk + 4 + g4], a1);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int at = (i0 + r16) * LDV2 + 16 * u + 4 * g4 + e;
        Vp[at] = Us[at] - (a0[e] + a1[e]);
      }
    }
    __syncthreads();
    // Oᵀ[dv][i] = γ_i (S Qᵀ)[dv][i] + (V'ᵀ Mᵀ)[dv][i]; M is lower triangular, so tokens j < i0 + 16 only
    {
      f4 a0 = f4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll 8
      for (int kk = 0; kk < DK; kk += 8) {
        a0 = mfma4(Ss[(16 * u + r16) * LDF + kk + g4], Qs[(i0 + r16) * LDF + kk + g4], a0);
        a1 = mfma4(Ss[(16 * u + r16) * LDF + kk + 4 + g4], Qs[(i0 + r16) * LDF + kk + 4 + g4], a1);
      }
      f4 acc = (a0 + a1) * Gm[i0 + r16];
      for (int jj = 0; jj < i0 + 16; jj += 4)
        acc = mfma4(Vp[(jj + g4) * LDV2 + 16 * u + r16], Ms[(i0 + r16) * LDM + jj + g4], acc);
      const uint32_t t = t0 + i0 + r16;
      if (t < T) {
        float* dst = o + ((size_t)t * NV + h) * DV + dv0 + 16 * u + 4 * g4;  // o need only be 4-byte aligned
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = acc[e];
      }
    }
    // S ← γ_C S + V'ᵀ diag(γ_C/γ) K on (value tile u, key tiles 2 (w / 2) + {0, 1})
    f4 sn[2];
    const float gC = Gm[C - 1];
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
      const int d0 = 16 * (2 * (wave >> 1) + q2);
#pragma unroll
      for (int e = 0; e < 4; ++e) sn[q2][e] = gC * Ss[(16 * u + 4 * g4 + e) * LDF + d0 + r16];
#pragma unroll 4
      for (int jj = 0; jj < C; jj += 4) {
        const int j = jj + g4;
        sn[q2] = mfma4(Vp[j * LDV2 + 16 * u + r16], Ks[j * LDK + d0 + r16] * Rh[j], sn[q2]);
      }
    }
    __syncthreads();  // every wave is done reading S
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
      const int d0 = 16 * (2 * (wave >> 1) + q2);
#pragma unroll
      for (int e = 0; e < 4; ++e) Ss[(16 * u + 4 * g4 + e) * LDF + d0 + r16] = sn[q2][e];
    }
  }
  __syncthreads();
  if (write_state) {
    for (int e = tid; e < kScanRows * DK / 4; e += kScanThreads) {
      const int r = e >> 5, d4 = (e & 31) * 4;
      *(f4*)(state_out + ((size_t)h * DV + dv0 + r) * DK + d4) = *(const f4*)(Ss + r * LDF + d4);
    }
  }
}

size_t delta_chunk_ws_floats(uint32_t t) { return (size_t)((t + C - 1) / C) * NV * kWsStride; }

hipError_t launch_gated_delta_chunked(const float* q, const float* k, const float* v, const float* a, const float* b,
                                      const float* a_log, const float* dt_bias, const float* state_in,
                                      float* state_out, float* o, float* ws, uint32_t t, uint32_t ldab,
                                      bool write_state, hipStream_t s) {
  const uint32_t nch = (t + C - 1) / C;
  hipLaunchKernelGGL(delta_chunk_prep_kernel, dim3(nch, NV), dim3(256), 0, s, q, k, v, a, b, ldab, a_log, dt_bias, ws,
                     t);
  hipLaunchKernelGGL(delta_chunk_scan_kernel, dim3(NV, DV / kScanRows), dim3(kScanThreads), 0, s, q, k, ws, state_in, state_out, o, t,
                     write_state ? 1u : 0u);
  return hipGetLastError();
}

}  // namespace dh
