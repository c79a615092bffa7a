// Row kernels around the GEMMs: the bitwise row gathers, the candidate-only
// LM head, the fp32 → fp16 row RMSNorm that produces every in-projection's
// activation, and the counter-based N(0, σ) fill used for random-init weights.
//
// decide counterparts: kernels/head.metal:8-59 (gather_rows_f32/f16,
// final_head), kernels/rmsnorm.metal:8-30 (rmsnorm_rows). All are HBM- or
// latency-bound; wave64 shuffles for the reductions.
#include "dh_kernels.h"
#include "normal_gen.h"

namespace dh {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over a 256-thread workgroup; every thread gets the total. `sh` holds 4 floats.
__device__ __forceinline__ float block_sum256(float v, float* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  const float t = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return t;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// ---------------------------------------------------------------------------
// out[i] = x[rowmap[i]], bitwise. One workgroup per output row; 16-byte copies
// when the row is a whole number of 16-byte vectors, else element copies.
template <typename T>
__global__ void gather_rows_kernel(const T* __restrict__ x, const uint32_t* __restrict__ rowmap, T* __restrict__ out,
                                   uint32_t h) {
  const uint32_t i = blockIdx.x;
  const T* src = x + (size_t)rowmap[i] * h;
  T* dst = out + (size_t)i * h;
  constexpr uint32_t V = 16 / sizeof(T);
  const bool vec = (h % V) == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15) == 0;
  if (vec) {
    for (uint32_t c = threadIdx.x; c < h / V; c += blockDim.x) ((uint4*)dst)[c] = ((const uint4*)src)[c];
  } else {
    for (uint32_t c = threadIdx.x; c < h; c += blockDim.x) dst[c] = src[c];
  }
}

hipError_t launch_gather_rows(const void* x, const uint32_t* rowmap, void* out, uint32_t rows, uint32_t h,
                              uint32_t elem_bytes, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (elem_bytes == 4)
    hipLaunchKernelGGL(gather_rows_kernel<uint32_t>, dim3(rows), dim3(256), 0, s, (const uint32_t*)x, rowmap,
                       (uint32_t*)out, h);
  else
    hipLaunchKernelGGL(gather_rows_kernel<uint16_t>, dim3(rows), dim3(256), 0, s, (const uint16_t*)x, rowmap,
                       (uint16_t*)out, h);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Candidate head. Workgroup (r, q) serves answer row r, candidates
// 8q .. 8q + 7: it recomputes the row's RMSNorm into LDS (fp32, cheap next to
// the table reads), then each wave takes two candidates and streams both bf16
// table rows with 16-byte loads, interleaved so two rows' loads are in flight.
// Splitting the candidates over workgroups puts rows × ⌈max_cand / 8⌉
// workgroups on the chip instead of one per row. Every candidate's sum is
// formed in the same order whatever the split (lane-strided, then a wave sum).
constexpr uint32_t kHeadCandPerGroup = 8;

__global__ __launch_bounds__(256) void final_head_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         const uint16_t* __restrict__ table,
                                                         const uint32_t* __restrict__ cand,
                                                         const uint32_t* __restrict__ ncand,
                                                         float* __restrict__ logits, uint32_t hidden,
                                                         uint32_t max_cand, float eps) {
  extern __shared__ float hn[];  // [hidden]
  __shared__ float sh[4];
  const uint32_t r = blockIdx.x;
  const uint32_t n = min(ncand[r], max_cand);
  const uint32_t c0 = blockIdx.y * kHeadCandPerGroup;
  if (c0 >= n) return;  // uniform over the workgroup
  const float* xr = x + (size_t)r * hidden;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < hidden; i += 256) {
    const float v = xr[i];
    ss += v * v;
  }
  const float inv = rsqrtf(block_sum256(ss, sh) / (float)hidden + eps);
  for (uint32_t i = threadIdx.x; i < hidden; i += 256) hn[i] = xr[i] * inv * (1.0f + w[i]);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t ca = c0 + 2 * wave, cb = ca + 1;
  if (ca >= n) return;
  const bool two = cb < n;
  const uint16_t* ea = table + (size_t)cand[(size_t)r * max_cand + ca] * hidden;
  const uint16_t* eb = two ? table + (size_t)cand[(size_t)r * max_cand + cb] * hidden : ea;
  float acc_a = 0.f, acc_b = 0.f;
  for (uint32_t i = lane * 8; i < hidden; i += 64 * 8) {
    const uint4 va = *(const uint4*)(ea + i);
    const uint4 vb = *(const uint4*)(eb + i);
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float h0 = hn[i + 2 * q], h1 = hn[i + 2 * q + 1];
      acc_a += h0 * bf16_to_f32((uint16_t)(wa[q] & 0xffffu));
      acc_a += h1 * bf16_to_f32((uint16_t)(wa[q] >> 16));
      acc_b += h0 * bf16_to_f32((uint16_t)(wb[q] & 0xffffu));
      acc_b += h1 * bf16_to_f32((uint16_t)(wb[q] >> 16));
    }
  }
  acc_a = wave_sum(acc_a);
  acc_b = wave_sum(acc_b);
  if (lane == 0) {
    logits[(size_t)r * max_cand + ca] = acc_a;
    if (two) logits[(size_t)r * max_cand + cb] = acc_b;
  }
}

hipError_t launch_final_head(const float* x, const float* w, const uint16_t* table, const uint32_t* cand,
                             const uint32_t* ncand, float* logits, uint32_t rows, uint32_t hidden, uint32_t max_cand,
                             float eps, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  const uint32_t groups = (max_cand + kHeadCandPerGroup - 1) / kHeadCandPerGroup;
  hipLaunchKernelGGL(final_head_kernel, dim3(rows, groups), dim3(256), hidden * sizeof(float), s, x, w, table, cand,
                     ncand, logits, hidden, max_cand, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// y[r] = half(x[rowmap[r]] · rsqrt(mean(x²) + eps) · w'), w' = 1 + w or w
// (rowmap NULL: row r itself).
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           _Float16* __restrict__ y,
                                                           const uint32_t* __restrict__ rowmap, uint32_t h,
                                                           uint32_t ld_in, uint32_t ld_out, uint32_t add_one,
                                                           float eps) {
  __shared__ float sh[4];
  const float* xr = x + (size_t)(rowmap ? rowmap[blockIdx.x] : blockIdx.x) * ld_in;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < h; i += 256) {
    const float v = xr[i];
    ss += v * v;
  }
  const float inv = rsqrtf(block_sum256(ss, sh) / (float)h + eps);
  _Float16* yr = y + (size_t)blockIdx.x * ld_out;
  for (uint32_t i = threadIdx.x; i < h; i += 256) {
    const float wv = add_one ? 1.0f + w[i] : w[i];
    yr[i] = (_Float16)(xr[i] * inv * wv);
  }
}

// The same norm with one wave per two rows for 16-byte-aligned rows of
// h % 4 == 0, h <= 256·KV: each row is loaded once into registers (KV float4
// per lane, all loads of both rows and of the weights in flight together),
// summed in the lane then across the wave, and written as half4. Eight rows
// per workgroup.
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// One float4's term of a row's sum of squares, and one float4 of the normed
// row: the arithmetic of every vectorised norm here, so they store the same
// bits. The pairs' fused multiply-adds are written out: left to the compiler,
// which product of a pair it fuses differed between kernels.
__device__ __forceinline__ float sq4(const f4& v) { return fmaf(v[0], v[0], v[1] * v[1]) + fmaf(v[2], v[2], v[3] * v[3]); }
__device__ __forceinline__ f4 weight4(const float* __restrict__ w, uint32_t i, uint32_t add_one) {
  f4 wv = *(const f4*)(w + 4 * i);
  if (add_one) wv += 1.0f;
  return wv;
}
__device__ __forceinline__ h4 norm4w(const f4& v, float inv, const f4& wv) {
  const f4 o = v * inv * wv;
  return h4{(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
}
__device__ __forceinline__ h4 norm4(const f4& v, float inv, const float* __restrict__ w, uint32_t i, uint32_t add_one) {
  return norm4w(v, inv, weight4(w, i, add_one));
}

template <int KV>
__global__ __launch_bounds__(256) void rmsnorm_rows_vec_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                               _Float16* __restrict__ y,
                                                               const uint32_t* __restrict__ rowmap, uint32_t rows,
                                                               uint32_t h, uint32_t ld_in, uint32_t ld_out,
                                                               uint32_t add_one, float eps) {
  // two rows per wave: the weights are loaded once for both, and both rows' loads are in flight together
  const uint32_t row0 = 2 * (blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row0 >= rows) return;
  const uint32_t lane = threadIdx.x & 63, n4 = h / 4;
  const bool two = row0 + 1 < rows;
  const float* xr0 = x + (size_t)(rowmap ? rowmap[row0] : row0) * ld_in;
  const float* xr1 = two ? x + (size_t)(rowmap ? rowmap[row0 + 1] : row0 + 1) * ld_in : xr0;
  f4 v0[KV], v1[KV], wv[KV];
#pragma unroll
  for (int q = 0; q < KV; ++q) {
    const uint32_t i = lane + 64 * q;
    v0[q] = i < n4 ? *(const f4*)(xr0 + 4 * i) : f4{0.f, 0.f, 0.f, 0.f};
    v1[q] = i < n4 ? *(const f4*)(xr1 + 4 * i) : f4{0.f, 0.f, 0.f, 0.f};
    wv[q] = i < n4 ? weight4(w, i, add_one) : f4{0.f, 0.f, 0.f, 0.f};
  }
  float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
  for (int q = 0; q < KV; ++q) {
    ss0 += sq4(v0[q]);
    ss1 += sq4(v1[q]);
  }
  const float inv0 = rsqrtf(wave_sum(ss0) / (float)h + eps);
  const float inv1 = rsqrtf(wave_sum(ss1) / (float)h + eps);
  _Float16* yr0 = y + (size_t)row0 * ld_out;
  _Float16* yr1 = yr0 + ld_out;
#pragma unroll
  for (int q = 0; q < KV; ++q) {
    const uint32_t i = lane + 64 * q;
    if (i < n4) {
      *(h4*)(yr0 + 4 * i) = norm4w(v0[q], inv0, wv[q]);
      if (two) *(h4*)(yr1 + 4 * i) = norm4w(v1[q], inv1, wv[q]);
    }
  }
}

// The residual add of a split-K projection fused with the norm that follows it:
//   x[r] += Σ_s ws[s][r]   (the partials summed in split order, then added to the row: splitk_reduce_kernel's AddF32)
//   y[r] = half(x[r] · rsqrt(mean(x[r]²) + eps) · w')   (rmsnorm_rows_vec_kernel<KV>'s arithmetic)
// One workgroup of 32·KV threads per row, two float4s per thread, every load of the row (S partials and the
// residual) in flight at once. The sum of squares keeps the vectorised norm's order: each float4's sq4 term goes
// to LDS, and lane l of wave 0 adds the terms of float4s l, l + 64, ... in that order before the wave sum, so x
// and y are bitwise those of the reduce followed by the norm.
template <int KV, int S>
__global__ __launch_bounds__(32 * KV) void splitk_add_rmsnorm_kernel(const float* __restrict__ ws, uint32_t rows,
                                                                     uint32_t h, float* __restrict__ x, uint32_t ldx,
                                                                     const float* __restrict__ w,
                                                                     _Float16* __restrict__ y, uint32_t ldy,
                                                                     uint32_t add_one, float eps) {
  constexpr uint32_t NT = 32 * KV;
  __shared__ float sq[64 * KV];
  __shared__ float sinv;
  const uint32_t row = blockIdx.x, t = threadIdx.x, n4 = h / 4;
  const size_t plane = (size_t)rows * h;
  const float* pr = ws + (size_t)row * h;
  float* xr = x + (size_t)row * ldx;
  f4 p[S][2], v[2], wv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t i = t + NT * j;
#pragma unroll
    for (int s = 0; s < S; ++s) p[s][j] = i < n4 ? *(const f4*)(pr + s * plane + 4 * i) : f4{0.f, 0.f, 0.f, 0.f};
    v[j] = i < n4 ? *(const f4*)(xr + 4 * i) : f4{0.f, 0.f, 0.f, 0.f};
    wv[j] = i < n4 ? weight4(w, i, add_one) : f4{0.f, 0.f, 0.f, 0.f};  // with the row: no load after the barriers
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t i = t + NT * j;
    f4 a = p[0][j];
#pragma unroll
    for (int s = 1; s < S; ++s) a += p[s][j];
    v[j] = a + v[j];
    if (i < n4) *(f4*)(xr + 4 * i) = v[j];
    sq[i] = i < n4 ? sq4(v[j]) : 0.f;
  }
  __syncthreads();
  if (t < 64) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < KV; ++q) ss += sq[t + 64 * q];
    const float inv = rsqrtf(wave_sum(ss) / (float)h + eps);
    if (t == 0) sinv = inv;
  }
  __syncthreads();
  const float inv = sinv;
  _Float16* yr = y + (size_t)row * ldy;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t i = t + NT * j;
    if (i < n4) *(h4*)(yr + 4 * i) = norm4w(v[j], inv, wv[j]);
  }
}

bool splitk_add_rmsnorm_fits(uint32_t splits, uint32_t h, uint32_t ldx, uint32_t ldy, const void* x, const void* w,
                             const void* y) {
  // the rows launch_rmsnorm_rows gives to rmsnorm_rows_vec_kernel<10>
  return splits >= 2 && splits <= 8 && h % 4 == 0 && h >= 4 && h <= 256 * 10 && ldx % 4 == 0 && ldy % 4 == 0 &&
         (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)y % 8 == 0;
}

hipError_t launch_splitk_add_rmsnorm(const float* ws, uint32_t splits, uint32_t rows, uint32_t h, float* x,
                                     uint32_t ldx, const float* w, _Float16* y, uint32_t ldy, bool add_one, float eps,
                                     hipStream_t s) {
  if (rows == 0) return hipSuccess;
  const uint32_t a1 = add_one ? 1u : 0u;
#define DH_ADDNORM(S_)                                                                                           \
  case S_:                                                                                                       \
    hipLaunchKernelGGL((splitk_add_rmsnorm_kernel<10, S_>), dim3(rows), dim3(320), 0, s, ws, rows, h, x, ldx, w, y, \
                       ldy, a1, eps);                                                                            \
    break;
  switch (splits) {
    DH_ADDNORM(2)
    DH_ADDNORM(3)
    DH_ADDNORM(4)
    DH_ADDNORM(5)
    DH_ADDNORM(6)
    DH_ADDNORM(7)
    DH_ADDNORM(8)
    default:
      return hipErrorInvalidValue;
  }
#undef DH_ADDNORM
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float* x, const float* w, _Float16* y, const uint32_t* rowmap, uint32_t rows,
                               uint32_t h, uint32_t ld_in, uint32_t ld_out, bool add_one, float eps, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  const bool vec = h % 4 == 0 && h <= 256 * 16 && ld_in % 4 == 0 && ld_out % 4 == 0 && (uintptr_t)x % 16 == 0 &&
                   (uintptr_t)w % 16 == 0 && (uintptr_t)y % 8 == 0;
  if (vec) {
    const dim3 grid((rows + 7) / 8);
    if (h <= 256 * 10)
      hipLaunchKernelGGL(rmsnorm_rows_vec_kernel<10>, grid, dim3(256), 0, s, x, w, y, rowmap, rows, h, ld_in, ld_out,
                         add_one ? 1u : 0u, eps);
    else
      hipLaunchKernelGGL(rmsnorm_rows_vec_kernel<16>, grid, dim3(256), 0, s, x, w, y, rowmap, rows, h, ld_in, ld_out,
                         add_one ? 1u : 0u, eps);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, s, x, w, y, rowmap, h, ld_in, ld_out,
                     add_one ? 1u : 0u, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// N(0, σ) fill rounded to fp16: element i is normal_at(seed, i) (normal_gen.h),
// so it depends only on (seed, i) and a host can reproduce its bits.
__global__ void fill_normal_f16_kernel(uint16_t* __restrict__ out, uint64_t n, uint64_t seed, float sd) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float z = normal_at(seed, i, 0.0f, sd);
    const _Float16 hv = (_Float16)z;
    out[i] = __builtin_bit_cast(uint16_t, hv);
  }
}

hipError_t launch_fill_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, float sd, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(fill_normal_f16_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, out, n, seed, sd);
  return hipGetLastError();
}

}  // namespace dh
