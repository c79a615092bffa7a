// The non-GEMM kernels of decide's hybrid decoder forward, for gfx950:
//   conv_silu_l2 / conv_state_update  (kernels/conv.metal; cpu_ref.rs:55-95)
//   gated_delta                       (kernels/delta_fast.metal; cpu_ref.rs:101-129)
//   gated_rmsnorm_silu                (kernels/gnorm.metal; cpu_ref.rs:132-145)
//   q_norm_rope / kv_norm_rope        (kernels/rope.metal; cpu_ref.rs:149-162)
//   embed_bf16                        (kernels/embed.metal)
//   fill_normal                       (random-init parameters of any dtype)
// Model constants are decide's (config.rs:4-31). Every kernel but the
// recurrence is HBM- or latency-bound; the recurrence is sequential over
// tokens and bound by its per-token dependency chain.
#include <type_traits>

#include "conv_common.h"
#include "dh_kernels.h"
#include "normal_gen.h"

namespace dh {

namespace {

constexpr int NK = 16, DK = 128, NV = 32, DV = 128;
constexpr int KEY_DIM = NK * DK, VALUE_DIM = NV * DV, CONV_DIM = 2 * KEY_DIM + VALUE_DIM;
constexpr int HEAD_DIM = 256, ROT_HALF = 32;

typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// silu and sigmoid with the hardware exp (decide uses fast-math exp for both,
// common.h:5-8); softplus with the precise exp/log (common.h:9-10).
__device__ __forceinline__ float silu_fast(float v) { return v / (1.0f + __expf(-v)); }
__device__ __forceinline__ float sigmoid_precise(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float softplus_precise(float v) { return v > 20.0f ? v : logf(1.0f + expf(v)); }

// Sum over each 16-lane row of the wave with DPP (xor 1, xor 2, half-row
// mirror, row mirror); every lane of the row ends with the same bits.
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

}  // namespace

// ---------------------------------------------------------------------------
// conv + SiLU + L2. One wave per (slot, run of 16 rows): slots 0-15 are q
// heads, 16-31 k heads, 32-63 v heads (128 channels each); lane l owns
// channels 2l, 2l + 1 of the slot. The arithmetic is conv_common.h's, which
// the chunked recurrence's prep kernel evaluates too when it fuses this step. The wave loads the run's 16 rows and the 3
// before it once (raw rows before the chunk come from `prev` [3][CONV_DIM]),
// all loads in flight together, and slides the 4-tap window over them; each
// output is the same fma chain as a single-row evaluation. Grid: (64 slots,
// runs of 64 rows), 4 waves per workgroup each taking 16 of them.
constexpr int kConvRun = 16;

__global__ __launch_bounds__(256) void conv_silu_l2_kernel(const float* __restrict__ p, const float* __restrict__ prev,
                                                           const float* __restrict__ w, float* __restrict__ q,
                                                           float* __restrict__ k, float* __restrict__ v, uint32_t T,
                                                           uint32_t ldp) {
  const uint32_t slot = blockIdx.x, lane = threadIdx.x & 63;
  const uint32_t t0 = blockIdx.y * 64 + (threadIdx.x >> 6) * kConvRun;
  if (t0 >= T) return;
  const uint32_t c = slot * 128 + 2 * lane;  // slots are laid out q | k | v along the qkv columns
  const f4 w0 = *(const f4*)(w + (size_t)c * 4), w1 = *(const f4*)(w + (size_t)(c + 1) * 4);
  f2 x[kConvRun + 3];  // raw rows t0 - 3 .. t0 + 15
#pragma unroll
  for (int j = 0; j < kConvRun + 3; ++j) {
    const int s = (int)t0 - 3 + j;
    if (s < 0)
      x[j] = *(const f2*)(prev + (size_t)(3 + s) * CONV_DIM + c);
    else
      x[j] = (uint32_t)s < T ? *(const f2*)(p + (size_t)s * ldp + c) : f2{0.f, 0.f};
  }
#pragma unroll
  for (int u = 0; u < kConvRun; ++u) {
    const uint32_t t = t0 + u;
    if (t >= T) break;
    const float y0 = convk::conv_silu(w0, x[u][0], x[u + 1][0], x[u + 2][0], x[u + 3][0]);
    const float y1 = convk::conv_silu(w1, x[u][1], x[u + 1][1], x[u + 2][1], x[u + 3][1]);
    if (slot >= 32) {
      *(f2*)(v + ((size_t)t * NV + (slot - 32)) * DV + 2 * lane) = f2{y0, y1};
      continue;
    }
    const float inv = convk::l2_inv(y0, y1);
    if (slot < 16) {
      const float sc = convk::q_scale(inv);
      *(f2*)(q + ((size_t)t * NK + slot) * DK + 2 * lane) = f2{y0 * sc, y1 * sc};
    } else {
      *(f2*)(k + ((size_t)t * NK + (slot - 16)) * DK + 2 * lane) = f2{y0 * inv, y1 * inv};
    }
  }
}

hipError_t launch_conv_silu_l2(const float* p, const float* prev, const float* w, float* q, float* k, float* v,
                               uint32_t t, uint32_t ldp, hipStream_t s) {
  if (t == 0) return hipSuccess;
  hipLaunchKernelGGL(conv_silu_l2_kernel, dim3(64, (t + 63) / 64), dim3(256), 0, s, p, prev, w, q, k, v, t, ldp);
  return hipGetLastError();
}

// out[i] = raw row t − 3 + i (from p if ≥ 0, else from prev_in). Each thread
// reads its channel's three sources before writing, so out may be prev_in.
__global__ void conv_state_update_kernel(const float* __restrict__ p, const float* prev_in, float* prev_out,
                                         uint32_t t, uint32_t ldp) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= (uint32_t)CONV_DIM) return;
  float r[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int s = (int)t - 3 + i;
    r[i] = s >= 0 ? p[(size_t)s * ldp + c] : prev_in[(size_t)(3 + s) * CONV_DIM + c];
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) prev_out[(size_t)i * CONV_DIM + c] = r[i];
}

hipError_t launch_conv_state_update(const float* p, const float* prev_in, float* prev_out, uint32_t t, uint32_t ldp,
                                    hipStream_t s) {
  hipLaunchKernelGGL(conv_state_update_kernel, dim3(CONV_DIM / 256), dim3(256), 0, s, p, prev_in, prev_out, t, ldp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gated delta recurrence. Lane l of a wave owns value row dv = 4·wave_in_group
// + l / 16 of head h and the key slice dk ∈ [8 (l % 16), +8): 8 floats of
// state in registers. Per token the two dot products (S·k and S·q) finish
// with a 16-lane DPP sum, so a token costs ~24 FMAs and 8 DPP adds per lane
// and no LDS, no barrier. The decay is a running scalar (S = c·S̃, c
// renormalised into S̃ below 2^-60), the form decide's fast kernel uses; c
// and 1/c depend on the gates only, so they stay off the per-token chain.
//
// Memory stays off the chain too. Tokens run in blocks of 64, each block's
// body fully unrolled: k, q, v of token t + 4 are loaded (index clamped, no
// branch) while token t computes; g and β of the next block are loaded one
// block ahead and computed lane-parallel (lane l ↔ token l) at the block
// start, then read per token with readlane; each row's 64 outputs are kept
// in registers (lane j holds tokens j, j+16, j+32, j+48) and written once per
// block. So the only stores, and the only full memory waits, come once per
// 64 tokens. Grid: (NV heads) × (DV / 16) workgroups of 256 threads.
constexpr int kDeltaPF = 4;
constexpr int kDeltaBlock = 64;
constexpr float kDeltaCMin = 8.673617e-19f;  // 2^-60

namespace {
struct DeltaLane {
  const float* __restrict__ q;
  const float* __restrict__ k;
  const float* __restrict__ v;
  uint32_t T, h, hk, dv, j;
  f4 kr[kDeltaPF][2], qr[kDeltaPF][2];
  float vr[kDeltaPF];
  float s[8];
  float c;

  __device__ __forceinline__ void load(uint32_t t, int slot) {
    t = min(t, T - 1);
    const f4* kp = (const f4*)(k + ((size_t)t * NK + hk) * DK + 8 * j);
    const f4* qp = (const f4*)(q + ((size_t)t * NK + hk) * DK + 8 * j);
    kr[slot][0] = kp[0];
    kr[slot][1] = kp[1];
    qr[slot][0] = qp[0];
    qr[slot][1] = qp[1];
    vr[slot] = v[((size_t)t * NV + h) * DV + dv];
  }

  // One token: consumes ring slot `slot`, refills it with token t + PF; returns o (every lane of the row).
  __device__ __forceinline__ float step(uint32_t t, int slot, float g, float beta) {
    const f4 k0 = kr[slot][0], k1 = kr[slot][1], q0 = qr[slot][0], q1 = qr[slot][1];
    const float vt = vr[slot];
    load(t + kDeltaPF, slot);
    float cg = c * g;
    if (cg < kDeltaCMin) {  // fold the scale into the state (uniform over the wave)
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] = (s[i] * c) * g;
      cg = 1.0f;
    }
    const float icg = __builtin_amdgcn_rcpf(cg);  // hardware reciprocal, as decide's fast-math division
    float ka = s[0] * k0[0], kb = s[4] * k1[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      ka = fmaf(s[i], k0[i], ka);
      kb = fmaf(s[4 + i], k1[i], kb);
    }
    const float kv = row16_sum(ka + kb);
    const float ds = (vt - cg * kv) * beta * icg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = fmaf(k0[i], ds, s[i]);
      s[4 + i] = fmaf(k1[i], ds, s[4 + i]);
    }
    float oa = s[0] * q0[0], ob = s[4] * q1[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      oa = fmaf(s[i], q0[i], oa);
      ob = fmaf(s[4 + i], q1[i], ob);
    }
    c = cg;
    return row16_sum(oa + ob) * cg;
  }
};

template <int B, int E, typename Fn>
__device__ __forceinline__ void unroll(Fn&& fn) {
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    unroll<B + 1, E>(fn);
  }
}
}  // namespace

__global__ __launch_bounds__(256) void gated_delta_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, const float* __restrict__ a,
                                                          const float* __restrict__ b, const float* __restrict__ a_log,
                                                          const float* __restrict__ dt_bias, const float* state_in,
                                                          float* state_out, float* __restrict__ o, uint32_t T,
                                                          uint32_t ldab, uint32_t write_state) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  DeltaLane L;
  L.q = q;
  L.k = k;
  L.v = v;
  L.T = T;
  L.h = blockIdx.x;
  L.hk = L.h >> 1;
  L.dv = blockIdx.y * 16 + wave * 4 + (lane >> 4);
  L.j = lane & 15;
  L.c = 1.0f;
  {
    const f4* src = (const f4*)(state_in + ((size_t)L.h * DV + L.dv) * DK + 8 * L.j);
    const f4 s0 = src[0], s1 = src[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      L.s[i] = s0[i];
      L.s[4 + i] = s1[i];
    }
  }
  const float A = expf(a_log[L.h]);
  const float bias = dt_bias[L.h];
  // gate inputs of the first block: lane l ↔ token l (clamped)
  float av = a[(size_t)min((uint32_t)lane, T - 1) * ldab + L.h];
  float bv = b[(size_t)min((uint32_t)lane, T - 1) * ldab + L.h];
#pragma unroll
  for (int i = 0; i < kDeltaPF; ++i) L.load(i, i);

  for (uint32_t t0 = 0; t0 < T; t0 += kDeltaBlock) {
    const float gv = expf(-A * softplus_precise(av + bias));
    const float bt = sigmoid_precise(bv);
    {  // next block's gate inputs, one block ahead
      const uint32_t tn = min(t0 + kDeltaBlock + lane, T - 1);
      av = a[(size_t)tn * ldab + L.h];
      bv = b[(size_t)tn * ldab + L.h];
    }
    float keep[4] = {0.f, 0.f, 0.f, 0.f};  // lane j: tokens t0 + j, + 16, + 32, + 48 of its row
    auto body = [&](auto guard) {
      unroll<0, kDeltaBlock>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if constexpr (decltype(guard)::value) {
          if (t0 + u >= T) return;
        }
        const float g = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gv), u));
        const float beta = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bt), u));
        const float ov = L.step(t0 + u, u % kDeltaPF, g, beta);
        if (L.j == (uint32_t)(u % 16)) keep[u / 16] = ov;
      });
    };
    // full blocks run straight-line code (exact wait counts); only the last block checks T
    if (t0 + kDeltaBlock <= T)
      body(std::false_type{});
    else
      body(std::true_type{});
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t t = t0 + 16 * r + L.j;
      if (t < T) o[((size_t)t * NV + L.h) * DV + L.dv] = keep[r];
    }
  }
  if (write_state) {
    f4* dst = (f4*)(state_out + ((size_t)L.h * DV + L.dv) * DK + 8 * L.j);
    const float c = L.c;
    dst[0] = f4{L.s[0] * c, L.s[1] * c, L.s[2] * c, L.s[3] * c};
    dst[1] = f4{L.s[4] * c, L.s[5] * c, L.s[6] * c, L.s[7] * c};
  }
}

hipError_t launch_gated_delta(const float* q, const float* k, const float* v, const float* a, const float* b,
                              const float* a_log, const float* dt_bias, const float* state_in, float* state_out,
                              float* o, uint32_t t, uint32_t ldab, bool write_state, hipStream_t s) {
  hipLaunchKernelGGL(gated_delta_kernel, dim3(NV, DV / 16), dim3(256), 0, s, q, k, v, a, b, a_log, dt_bias, state_in,
                     state_out, o, t, ldab, write_state ? 1u : 0u);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gated RMSNorm: one wave per (row, value head), lane l owns dims 2l, 2l + 1.
// y = half(o · rsqrt(mean(o²) + eps) · w · silu(z)). Grid (NV / 4, T) × 256.
__global__ __launch_bounds__(256) void gated_rmsnorm_silu_kernel(const float* __restrict__ o,
                                                                 const float* __restrict__ z,
                                                                 const float* __restrict__ w, _Float16* __restrict__ y,
                                                                 uint32_t ldz) {
  const int lane = threadIdx.x & 63;
  const uint32_t h = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y;
  const f2 x = *(const f2*)(o + ((size_t)t * NV + h) * DV + 2 * lane);
  const float inv = rsqrtf(wave_sum(x[0] * x[0] + x[1] * x[1]) / (float)DV + 1e-6f);
  const uint32_t d = 2 * lane;
  const f2 zz = *(const f2*)(z + (size_t)t * ldz + h * DV + d);
  const f2 ww = *(const f2*)(w + d);
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  *(h2*)(y + (size_t)t * VALUE_DIM + h * DV + d) =
      h2{(_Float16)(x[0] * inv * ww[0] * silu_fast(zz[0])), (_Float16)(x[1] * inv * ww[1] * silu_fast(zz[1]))};
}

hipError_t launch_gated_rmsnorm_silu(const float* o, const float* z, const float* w, _Float16* y, uint32_t t,
                                     uint32_t ldz, hipStream_t s) {
  if (t == 0) return hipSuccess;
  hipLaunchKernelGGL(gated_rmsnorm_silu_kernel, dim3(NV / 4, t), dim3(256), 0, s, o, z, w, y, ldz);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Zero-centred RMSNorm over a 256-dim head, then RoPE on dims [0, 64) (pairs
// i, i + 32) at position pos. One wave per head; lane l owns dims 4l .. 4l+3,
// so lane l < 8 pairs with lane l + 8 (xor 8). Returns the lane's 4 values.
__device__ __forceinline__ f4 norm_rope4(f4 x, const float* __restrict__ wn, const float* __restrict__ inv_freq,
                                         uint32_t pos, int lane) {
  const float inv = rsqrtf(wave_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]) / (float)HEAD_DIM + 1e-6f);
  const f4 wv = *(const f4*)(wn + 4 * lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = x[i] * inv * (1.0f + wv[i]);
  f4 other;
#pragma unroll
  for (int i = 0; i < 4; ++i) other[i] = __shfl_xor(x[i], 8, 64);
  if (lane < 16) {
    const bool lo = lane < 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 4 * lane + i;
      const float ang = (float)pos * inv_freq[d % ROT_HALF];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      // lo: x = a (dim i), other = b (dim i + 32) → a·c − b·s; hi: x = b, other = a → b·c + a·s
      x[i] = lo ? x[i] * cs - other[i] * sn : x[i] * cs + other[i] * sn;
    }
  }
  return x;
}

// q heads: rows of pq (stride ldq), head h at column 256 h → qo fp16 [rows][16][256].
// Grid (4, rows) × 256: four heads per workgroup.
__global__ __launch_bounds__(256) void q_norm_rope_kernel(const float* __restrict__ pq, const float* __restrict__ qw,
                                                          const float* __restrict__ inv_freq,
                                                          const uint32_t* __restrict__ qpos, _Float16* __restrict__ qo,
                                                          uint32_t ldq) {
  const int lane = threadIdx.x & 63;
  const uint32_t h = blockIdx.x * 4 + (threadIdx.x >> 6), r = blockIdx.y;
  const f4 x = *(const f4*)(pq + (size_t)r * ldq + h * HEAD_DIM + 4 * lane);
  const f4 y = norm_rope4(x, qw, inv_freq, qpos[r], lane);
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  *(h4*)(qo + ((size_t)r * 16 + h) * HEAD_DIM + 4 * lane) = h4{(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
}

hipError_t launch_q_norm_rope(const float* pq, const float* qw, const float* inv_freq, const uint32_t* qpos,
                              _Float16* qo, uint32_t rows, uint32_t ldq, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(q_norm_rope_kernel, dim3(4, rows), dim3(256), 0, s, pq, qw, inv_freq, qpos, qo, ldq);
  return hipGetLastError();
}

// k heads (norm + RoPE) into kc and v heads (copied) into vc, fp16 caches
// [pos][4][256], position pos0 + r. Grid (2, rows) × 256: workgroup x = 0
// takes the 4 k heads, x = 1 the 4 v heads.
__global__ __launch_bounds__(256) void kv_norm_rope_kernel(const float* __restrict__ pkv, const float* __restrict__ kw,
                                                           const float* __restrict__ inv_freq, _Float16* __restrict__ kc,
                                                           _Float16* __restrict__ vc, uint32_t ldkv, uint32_t kcol,
                                                           uint32_t vcol, uint32_t pos0) {
  const int lane = threadIdx.x & 63;
  const uint32_t jh = threadIdx.x >> 6, r = blockIdx.y, pos = pos0 + r;
  const float* row = pkv + (size_t)r * ldkv;
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  if (blockIdx.x == 1) {
    const f4 x = *(const f4*)(row + vcol + jh * HEAD_DIM + 4 * lane);
    *(h4*)(vc + ((size_t)pos * 4 + jh) * HEAD_DIM + 4 * lane) = h4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
    return;
  }
  const f4 x = *(const f4*)(row + kcol + jh * HEAD_DIM + 4 * lane);
  const f4 y = norm_rope4(x, kw, inv_freq, pos, lane);
  *(h4*)(kc + ((size_t)pos * 4 + jh) * HEAD_DIM + 4 * lane) = h4{(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
}

hipError_t launch_kv_norm_rope(const float* pkv, const float* kw, const float* inv_freq, _Float16* kc, _Float16* vc,
                               uint32_t rows, uint32_t ldkv, uint32_t kcol, uint32_t vcol, uint32_t pos0,
                               hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_norm_rope_kernel, dim3(2, rows), dim3(256), 0, s, pkv, kw, inv_freq, kc, vc, ldkv, kcol, vcol,
                     pos0);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// out[t][c] = float(table[ids[t]][c]) (bf16 widened, bitwise). 8 columns per thread.
__global__ void embed_bf16_kernel(const uint32_t* __restrict__ ids, const uint16_t* __restrict__ table,
                                  float* __restrict__ out, uint32_t h) {
  const uint32_t t = blockIdx.y;
  const uint16_t* src = table + (size_t)ids[t] * h;
  float* dst = out + (size_t)t * h;
  for (uint32_t c = (blockIdx.x * blockDim.x + threadIdx.x) * 8; c < h; c += gridDim.x * blockDim.x * 8) {
    const uint4 u = *(const uint4*)(src + c);
    const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
    f4 lo, hi;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      lo[2 * i] = __uint_as_float(wv[i] << 16);
      lo[2 * i + 1] = __uint_as_float(wv[i] & 0xffff0000u);
      hi[2 * i] = __uint_as_float(wv[2 + i] << 16);
      hi[2 * i + 1] = __uint_as_float(wv[2 + i] & 0xffff0000u);
    }
    *(f4*)(dst + c) = lo;
    *(f4*)(dst + c + 4) = hi;
  }
}

hipError_t launch_embed_bf16(const uint32_t* ids, const uint16_t* table, float* out, uint32_t t, uint32_t h,
                             hipStream_t s) {
  if (t == 0) return hipSuccess;
  const uint32_t bx = (h / 8 + 255) / 256;
  hipLaunchKernelGGL(embed_bf16_kernel, dim3(bx, t), dim3(256), 0, s, ids, table, out, h);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// N(mean, σ) fill of fp16 (dtype 0), bf16 (1) or fp32 (2) values: element i is
// normal_at(seed, i, mean, σ) (normal_gen.h) rounded to nearest even.
__global__ void fill_normal_kernel(void* __restrict__ out, uint64_t n, uint64_t seed, float mean, float sd,
                                   uint32_t dtype) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float zv = normal_at(seed, i, mean, sd);
    if (dtype == 0) {
      ((_Float16*)out)[i] = (_Float16)zv;
    } else if (dtype == 1) {
      const uint32_t u = __float_as_uint(zv);
      ((uint16_t*)out)[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);  // RNE (finite inputs)
    } else {
      ((float*)out)[i] = zv;
    }
  }
}

hipError_t launch_fill_normal(void* out, uint64_t n, uint64_t seed, float mean, float sd, uint32_t dtype,
                              hipStream_t s) {
  if (n == 0) return hipSuccess;
  const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(fill_normal_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, out, n, seed, mean, sd, dtype);
  return hipGetLastError();
}

}  // namespace dh
