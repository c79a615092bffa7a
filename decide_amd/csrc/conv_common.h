// The arithmetic of decide's causal conv + SiLU + L2 step (kernels/conv.metal;
// cpu_ref.rs:55-81), shared by the stand-alone conv kernel (mixer.hip) and the
// chunked recurrence's prep kernel that computes it on the fly
// (delta_chunk.hip): both evaluate every channel through these functions, so
// they produce the same bits.
#pragma once

#include <hip/hip_runtime.h>

namespace dh {
namespace convk {

constexpr int NK = 16, DK = 128, NV = 32, DV = 128;
constexpr int KEY_DIM = NK * DK, VALUE_DIM = NV * DV, CONV_DIM = 2 * KEY_DIM + VALUE_DIM;

typedef float f4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wave, every lane ending with the same bits: within
// each 16-lane row by DPP (xor 1, xor 2, half-row mirror, row mirror), then
// across rows with gfx950's swaps (permlane16_swap pairs rows 0-1 and 2-3,
// permlane32_swap the halves; called with the same value twice, the two
// results are the value and its partner's). No LDS round trip.
__device__ __forceinline__ float wave_sum64(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// silu with the hardware exp and reciprocal (decide uses fast-math exp for it,
// common.h:5-8).
__device__ __forceinline__ float silu_fast(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// One channel's output: the 4-tap causal conv over raw rows t - 3 .. t (x0 is
// row t - 3), accumulated in that order, then SiLU.
__device__ __forceinline__ float conv_silu(const f4& w, float x0, float x1, float x2, float x3) {
  float a = fmaf(w[0], x0, 0.f);
  a = fmaf(w[1], x1, a);
  a = fmaf(w[2], x2, a);
  a = fmaf(w[3], x3, a);
  return silu_fast(a);
}

// 1 / ‖row‖ of one 128-channel head whose lane l holds channels 2l and 2l + 1.
__device__ __forceinline__ float l2_inv(float y0, float y1) { return rsqrtf(wave_sum64(fmaf(y0, y0, y1 * y1)) + 1e-6f); }

// q's scale: 1 / ‖q‖ · DK^-1/2.
__device__ __forceinline__ float q_scale(float inv) { return inv * 0.08838834764831845f; }

}  // namespace convk
}  // namespace dh
