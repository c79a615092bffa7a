// Host-side weight layouts for the fused GEMM operands (include/decide_hip.h).
// decide builds these offline in its converter: deinterleave_q_gate,
// interleave_gate_up and bf16_to_f16 (crates/decide-engine/src/convert.rs:37-90).
// The permutations must be exactly decide's, because dh_gemm_nt's SwiGLU
// epilogue and the mixers downstream read columns at fixed offsets.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/decide_hip.h"

namespace {

// IEEE binary32 → binary16, round to nearest even (the `half` crate's
// f16::from_f32), written from the bit patterns.
uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {  // inf or nan
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: overflow
  if (ax < 0x38800000u) {  // below the smallest normal half (2^-14): subnormal or zero
    if (ax < 0x33000000u) return (uint16_t)sign;  // < 2^-25: rounds to zero
    const uint32_t e = ax >> 23;                   // biased exponent, 102..112
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;               // 14..24
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((ax >> 13) - (112u << 10));  // rebias exponent 127 → 15
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

}  // namespace

extern "C" {

int dh_interleave_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint32_t n, uint32_t k,
                          uint32_t block) {
  if (!gate || !up || !out || block == 0 || n % block != 0) return DH_EINVAL;
  const size_t row = (size_t)k;
  size_t o = 0;
  for (uint32_t b = 0; b < n / block; ++b) {
    std::memcpy(out + o, gate + (size_t)b * block * row, block * row * 2);
    o += block * row;
    std::memcpy(out + o, up + (size_t)b * block * row, block * row * 2);
    o += block * row;
  }
  return DH_OK;
}

int dh_deinterleave_q_gate(const uint16_t* src, uint16_t* out, uint32_t heads, uint32_t head_dim, uint32_t k) {
  if (!src || !out) return DH_EINVAL;
  const size_t span = (size_t)head_dim * k;
  size_t o = 0;
  for (uint32_t part = 0; part < 2; ++part)
    for (uint32_t h = 0; h < heads; ++h) {
      std::memcpy(out + o, src + ((size_t)h * 2 + part) * span, span * 2);
      o += span;
    }
  return DH_OK;
}

int dh_bf16_to_f16(const uint16_t* src, uint16_t* out, uint64_t n, uint64_t* counts) {
  if (n && (!src || !out)) return DH_EINVAL;
  uint64_t sub = 0, ftz = 0, ovf = 0;
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t bits = (uint32_t)src[i] << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    const uint16_t h = f32_to_f16_rne(f);
    out[i] = h;
    const uint16_t ah = h & 0x7fffu;
    if (ah == 0x7c00u && std::isfinite(f))
      ++ovf;
    else if (ah == 0 && f != 0.0f)
      ++ftz;
    else if (ah != 0 && ah < 0x0400u)
      ++sub;
  }
  if (counts) {
    counts[0] = n;
    counts[1] = sub;
    counts[2] = ftz;
    counts[3] = ovf;
  }
  return ovf ? DH_EINVAL : DH_OK;
}

}  // extern "C"
