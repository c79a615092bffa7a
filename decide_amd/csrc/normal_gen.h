// Seeded Gaussian generator shared by the library's fill kernels.
//
// Element i of the stream with seed s:
//   * two 24-bit uniforms from splitmix64's finaliser over s + φ·(2p + 1) and
//     s + φ·(2p + 2), p = i >> 1, φ = 0x9e3779b97f4a7c15 (mod 2⁶⁴);
//   * Box–Muller on that pair: r = sqrt(−2 ln u₁), θ = 2π u₂, with
//     u = (bits + ½)·2⁻²⁴; even i takes r·cos θ, odd i r·sin θ;
//   * value = (r·trig)·sd + mean in fp32, then rounded to the tensor's type.
//
// The arithmetic is fp32 with IEEE-rounded +, −, ×, ÷ and sqrt only, in one
// fixed order, and no contraction into fused multiply-adds, so any host that
// follows the same steps gets the same bits (hipcc lowers fp32 ÷ and sqrt to
// correctly rounded sequences for gfx950). The transcendental pieces are
// written out instead of calling the device math library:
//   * ln u₁: u₁ = m·2ᵉ with m in [√½, √2), ln m = 2·atanh(z), z = (m−1)/(m+1),
//     |z| ≤ 0.1716, summed as 2z·(1 + z²/3 + z⁴/5 + … + z¹⁰/11) (the dropped
//     term is below 1e-11); ln u₁ = ln m + e·ln 2;
//   * θ = (π/4)(o + t), octant o = the top 3 bits of u₂'s 24, t in (0, 1)
//     from the other 21 (exact); each octant is folded to an angle β with
//     |β| < π/4 and a quarter turn k, and sin β, cos β come from their Taylor
//     series in t to the (π/4)¹¹/11! and (π/4)¹²/12! terms.
#pragma once

#include <stdint.h>

namespace dh {

__device__ __forceinline__ uint64_t normal_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// ln u for u in (0, 1]: exponent split, then the atanh series (no libm).
// Constants are the fp32 roundings of 1/k, ln 2 and √2, written in hex.
__device__ __forceinline__ float normal_ln(float u) {
#pragma clang fp contract(off)
  const uint32_t bits = __float_as_uint(u);
  int e = (int)(bits >> 23) - 127;
  float m = __uint_as_float((bits & 0x7fffffu) | 0x3f800000u);
  if (m > 0x1.6a09e6p+0f) {
    m = m * 0.5f;
    e = e + 1;
  }
  const float z = (m - 1.0f) / (m + 1.0f);
  const float z2 = z * z;
  float p = 0x1.745d18p-4f;     // 1/11
  p = p * z2 + 0x1.c71c72p-4f;  // 1/9
  p = p * z2 + 0x1.24924ap-3f;  // 1/7
  p = p * z2 + 0x1.99999ap-3f;  // 1/5
  p = p * z2 + 0x1.555556p-2f;  // 1/3
  p = p * z2 + 1.0f;
  const float lnm = (z + z) * p;
  return (float)e * 0x1.62e430p-1f + lnm;
}

// sin((π/4)·t) and cos((π/4)·t) for t in [0, 1]: Taylor series in t, with
// coefficients the fp32 roundings of ±(π/4)ᵏ/k!, written in hex.
__device__ __forceinline__ void normal_sincos_octant(float t, float* s, float* c) {
#pragma clang fp contract(off)
  const float t2 = t * t;
  float ps = -0x1.e30750p-30f;   // k = 11
  ps = ps * t2 + 0x1.507834p-22f;  // k = 9
  ps = ps * t2 - 0x1.32d2ccp-15f;  // k = 7
  ps = ps * t2 + 0x1.466bc6p-9f;   // k = 5
  ps = ps * t2 - 0x1.4abbcep-4f;   // k = 3
  ps = ps * t2 + 0x1.921fb6p-1f;   // k = 1
  *s = t * ps;
  float pc = 0x1.f9d38ap-34f;     // k = 12
  pc = pc * t2 - 0x1.a6d1f2p-26f;  // k = 10
  pc = pc * t2 + 0x1.e1f506p-19f;  // k = 8
  pc = pc * t2 - 0x1.55d3c8p-12f;  // k = 6
  pc = pc * t2 + 0x1.03c1f0p-6f;   // k = 4
  pc = pc * t2 - 0x1.3bd3ccp-2f;   // k = 2
  pc = pc * t2 + 1.0f;
  *c = pc;
}

// Element i of the N(mean, sd) stream with seed `seed`, in fp32.
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i, float mean, float sd) {
#pragma clang fp contract(off)
  const uint64_t pidx = i >> 1;
  const uint32_t a = (uint32_t)(normal_mix64(seed + 0x9e3779b97f4a7c15ull * (2 * pidx + 1)) >> 40);
  const uint32_t b = (uint32_t)(normal_mix64(seed + 0x9e3779b97f4a7c15ull * (2 * pidx + 2)) >> 40);
  const float u1 = ((float)a + 0.5f) * 0x1p-24f;
  const float r = __builtin_sqrtf(-2.0f * normal_ln(u1));
  // θ = 2π(b + ½)/2²⁴ = (π/4)(o + t)
  const uint32_t o = b >> 21;
  const float t = ((float)(b & 0x1fffffu) + 0.5f) * 0x1p-21f;
  // even octant: θ = k·π/2 + (π/4)t with k = o/2; odd: θ = k·π/2 − (π/4)(1 − t) with k = (o + 1)/2
  float sb, cb;
  normal_sincos_octant((o & 1u) ? 1.0f - t : t, &sb, &cb);
  if (o & 1u) sb = -sb;
  const uint32_t k = ((o + 1u) >> 1) & 3u;
  float cth, sth;
  if (k == 0) {
    cth = cb;
    sth = sb;
  } else if (k == 1) {
    cth = -sb;
    sth = cb;
  } else if (k == 2) {
    cth = -cb;
    sth = -sb;
  } else {
    cth = sb;
    sth = -cb;
  }
  const float z = r * ((i & 1) ? sth : cth);
  return z * sd + mean;
}

}  // namespace dh
