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
// parallel; kernel 2 (scan) runs the chunks in order for each (head, 16 value
// rows). Tokens past T in the last chunk enter with k = q = v = 0, β = 0 and
// log g = 0, so they change nothing.
#include <type_traits>

#include "dh_kernels.h"

namespace dh {

namespace {

constexpr int C = 64;            // tokens per chunk
constexpr int NK = 16, DK = 128, NV = 32, DV = 128;
constexpr int LDF = DK + 4;      // fp32 row stride of the 64 × 128 LDS tiles (conflict-free MFMA operand reads)
constexpr int LDT = C + 1;       // row stride of the 64 × 64 triangular tiles
constexpr int LDM = C + 4;
constexpr int LDV = 16 + 1;
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

// Rows t0 .. t0 + 63 of a [T][heads][128] fp32 tensor (head `hd`) into an LDS tile (zero past T).
__device__ __forceinline__ void load_rows(float* dst, const float* __restrict__ src, uint32_t t0, uint32_t T,
                                          uint32_t heads, uint32_t hd, int tid) {
  for (int e = tid; e < C * DK / 4; e += 256) {
    const int i = e >> 5, d4 = (e & 31) * 4;
    const uint32_t t = t0 + i;
    f4 x = f4{0.f, 0.f, 0.f, 0.f};
    if (t < T) x = *(const f4*)(src + ((size_t)t * heads + hd) * DK + d4);
    *(f4*)(dst + i * LDF + d4) = x;
  }
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
  __shared__ __attribute__((aligned(16))) float Vs[C * LDF];
  __shared__ float As[C * LDT];
  __shared__ float Ts[C * LDT];
  __shared__ float Lg[C], Bt[C], Gm[C];
  const uint32_t c = blockIdx.x, h = blockIdx.y, hk = h >> 1, t0 = c * C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  float* out = ws + ((size_t)c * NV + h) * kWsStride;

  load_rows(Ks, k, t0, T, NK, hk, tid);
  load_rows(Qs, q, t0, T, NK, hk, tid);
  load_rows(Vs, v, t0, T, NV, h, tid);
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

  // K Kᵀ → A (strictly lower, β_i γ_i/γ_j), Q Kᵀ → M (lower incl. diagonal, γ_i/γ_j): 2 × 16 tiles of 16 × 16
  for (int tt = wave; tt < 32; tt += 4) {
    const bool isq = tt >= 16;
    const int ti = (tt & 15) >> 2, tj = tt & 3;
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
  __syncthreads();

  // T = (I + A)⁻¹ by forward substitution: lane j of wave 0 owns column j.
  if (wave == 0) {
    float x[C];
    sfor<0, C>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      float s = 0.f;
      sfor<0, i>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        s = fmaf(As[i * LDT + m], x[m], s);
      });
      x[i] = i == lane ? 1.0f : -s;  // x_m = 0 for m < lane, so rows above the diagonal stay 0
    });
    sfor<0, C>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      Ts[i * LDT + lane] = x[i];
    });
  }
  __syncthreads();

  // W = T diag(βγ) K and U = T diag(β) V: 2 × 32 tiles of 16 × 16 over K = 64
  for (int tt = wave; tt < 64; tt += 4) {
    const bool isu = tt >= 32;
    const int ti = (tt & 31) >> 3, td = tt & 7;
    const float* R = isu ? Vs : Ks;
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int jj = 0; jj < C; jj += 4) {
      const int j = jj + g4;
      const float sc = isu ? Bt[j] : Bt[j] * Gm[j];
      acc = mfma4(Ts[(16 * ti + r16) * LDT + j], R[j * LDF + 16 * td + r16] * sc, acc);
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

// One workgroup per (value head, 16 value rows); the state slice S [16][128]
// stays in LDS across all chunks. Wave w takes token tile w (16 tokens) for
// V' and O, and key-dim tiles 2w, 2w + 1 for the state update.
__global__ __launch_bounds__(256) void delta_chunk_scan_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                               const float* __restrict__ ws, const float* state_in,
                                                               float* state_out, float* __restrict__ o, uint32_t T,
                                                               uint32_t write_state) {
  __shared__ __attribute__((aligned(16))) float Ss[16 * LDF];
  __shared__ __attribute__((aligned(16))) float Ws[C * LDF];
  __shared__ __attribute__((aligned(16))) float Qs[C * LDF];
  __shared__ __attribute__((aligned(16))) float Ks[C * LDF];
  __shared__ float Ms[C * LDM];
  __shared__ float Us[C * LDV];
  __shared__ float Vp[C * LDV];
  __shared__ float Gm[C], Rh[C];
  const uint32_t h = blockIdx.x, hk = h >> 1, dv0 = blockIdx.y * 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;

  for (int e = tid; e < 16 * DK / 4; e += 256) {
    const int r = e >> 5, d4 = (e & 31) * 4;
    *(f4*)(Ss + r * LDF + d4) = *(const f4*)(state_in + ((size_t)h * DV + dv0 + r) * DK + d4);
  }
  const uint32_t nch = (T + C - 1) / C;
  for (uint32_t c = 0; c < nch; ++c) {
    const uint32_t t0 = c * C;
    const float* in = ws + ((size_t)c * NV + h) * kWsStride;
    __syncthreads();  // the previous chunk's reads of the staged tiles are done
    for (int e = tid; e < C * DK / 4; e += 256) {
      const int i = e >> 5, d4 = (e & 31) * 4;
      *(f4*)(Ws + i * LDF + d4) = *(const f4*)(in + kOffW + i * DK + d4);
    }
    load_rows(Qs, q, t0, T, NK, hk, tid);
    load_rows(Ks, k, t0, T, NK, hk, tid);
    for (int e = tid; e < C * C; e += 256) Ms[(e >> 6) * LDM + (e & 63)] = in[kOffM + e];
    for (int e = tid; e < C * 16; e += 256) Us[(e >> 4) * LDV + (e & 15)] = in[kOffU + (e >> 4) * DK + dv0 + (e & 15)];
    if (tid < C) {
      Gm[tid] = in[kOffGam + tid];
      Rh[tid] = in[kOffRho + tid];
    }
    __syncthreads();

    // V'ᵀ[dv][i] = Uᵀ − S Wᵀ for token tile i ∈ [16 w, 16 w + 16)
    const int i0 = 16 * wave;
    {
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int kk = 0; kk < DK; kk += 4) acc = mfma4(Ss[r16 * LDF + kk + g4], Ws[(i0 + r16) * LDF + kk + g4], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int dv = 4 * g4 + e, i = i0 + r16;
        Vp[i * LDV + dv] = Us[i * LDV + dv] - acc[e];
      }
    }
    __syncthreads();
    // Oᵀ[dv][i] = γ_i (S Qᵀ)[dv][i] + (V'ᵀ Mᵀ)[dv][i]
    {
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int kk = 0; kk < DK; kk += 4) acc = mfma4(Ss[r16 * LDF + kk + g4], Qs[(i0 + r16) * LDF + kk + g4], acc);
      acc *= Gm[i0 + r16];
#pragma unroll 4
      for (int jj = 0; jj < C; jj += 4) acc = mfma4(Vp[(jj + g4) * LDV + r16], Ms[(i0 + r16) * LDM + jj + g4], acc);
      const uint32_t t = t0 + i0 + r16;
      if (t < T) {
        float* dst = o + ((size_t)t * NV + h) * DV + dv0 + 4 * g4;  // o need only be 4-byte aligned
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = acc[e];
      }
    }
    // S ← γ_C S + V'ᵀ diag(γ_C/γ) K, key-dim tiles 2w and 2w + 1
    f4 sn[2];
    const float gC = Gm[C - 1];
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
      const int d0 = 16 * (2 * wave + q2);
      f4 acc;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = gC * Ss[(4 * g4 + e) * LDF + d0 + r16];
#pragma unroll 4
      for (int jj = 0; jj < C; jj += 4) {
        const int j = jj + g4;
        acc = mfma4(Vp[j * LDV + r16], Ks[j * LDF + d0 + r16] * Rh[j], acc);
      }
      sn[q2] = acc;
    }
    __syncthreads();  // every wave is done reading S
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
      const int d0 = 16 * (2 * wave + q2);
#pragma unroll
      for (int e = 0; e < 4; ++e) Ss[(4 * g4 + e) * LDF + d0 + r16] = sn[q2][e];
    }
  }
  __syncthreads();
  if (write_state) {
    for (int e = tid; e < 16 * DK / 4; e += 256) {
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
  hipLaunchKernelGGL(delta_chunk_scan_kernel, dim3(NV, DV / 16), dim3(256), 0, s, q, k, ws, state_in, state_out, o, t,
                     write_state ? 1u : 0u);
  return hipGetLastError();
}

}  // namespace dh
