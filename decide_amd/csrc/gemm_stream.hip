// Small-M weight-streaming GEMM for gfx950: Y = epi(X · Wᵀ) for M ≤ 16, the
// role of decide's `gemm_nt_small` (kernels/gemm_fast.metal:429-566). At this
// M the GEMM is a pass over W, bound by HBM; the design keeps every byte of W
// moving and nothing else in the way:
//   * A workgroup owns 32 output columns (two 16-column MFMA fragments, so the
//     SwiGLU gate|up blocks of decide's interleave stay together) and a K
//     range; its 4 waves take the range's 128-wide k blocks round-robin, so at
//     any moment they stream adjacent 256-byte runs of the same 32 W rows.
//   * W goes from HBM straight into registers: for k block b and MFMA step q,
//     lane (r, g) loads W[n0 + r][128 b + 32 q + 8 g .. + 8], 64 contiguous
//     bytes per row per instruction, which is the B operand of
//     v_mfma_f32_16x16x32_f16 as it stands. X rows (clamped to M − 1) come
//     from L2 the same way as the A operand.
//   * Loads run D k blocks ahead through a register ring. They are plain
//     vector loads, so the compiler sees every one and places the waits
//     before each register's first use itself.
//   * The 4 waves' partial sums meet in LDS and are added in wave order;
//     split-K across workgroups writes fp32 partials that
//     splitk_reduce_kernel sums in split order. Deterministic.
#include <type_traits>

#include "dh_kernels.h"

namespace dh {

namespace {
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kSK = 128;  // k per block
constexpr int kD = 3;     // k blocks in flight per wave

template <int B, int E, typename Fn>
__device__ __forceinline__ void sfor(Fn&& fn) {
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    sfor<B + 1, E>(fn);
  }
}

__device__ __forceinline__ void load16(h8& dst, const _Float16* src) { dst = *(const h8*)src; }

__device__ __forceinline__ f4 mfma16(const h8& a, const h8& b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// silu(g) · u in fp32, evaluated as the tile kernels evaluate it.
__device__ __forceinline__ float swiglu_f(float g, float u) { return silu_f(g) * u; }
}  // namespace

__global__ __launch_bounds__(256) void gemm_stream_kernel(const TileArgs a) {
  __shared__ f4 red[4][2][64];
  const uint32_t cb = blockIdx.x % a.nstripes, split = blockIdx.x / a.nstripes;
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxMembers; ++i)
    if (i < (int)a.count && cb >= a.mem[i].stripe_begin) mi = i;
  const Member& mb = a.mem[mi];
  const uint32_t n0 = (cb - mb.stripe_begin) * 32, N = mb.n, M = a.m;
  const uint32_t kb0 = split * a.kps, kend = min(a.k, kb0 + a.kps);
  const int nbk = (int)((kend - kb0) / kSK);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nbw = nbk > wave ? (nbk - wave + 3) / 4 : 0;  // this wave's blocks: wave, wave + 4, ...

  const _Float16* xr = a.x + (size_t)min((uint32_t)r, M - 1) * a.ldx + kb0 + 8 * g;
  const _Float16* w0 = mb.w + (size_t)min(n0 + r, N - 1) * mb.ldw + kb0 + 8 * g;
  const _Float16* w1 = mb.w + (size_t)min(n0 + 16 + r, N - 1) * mb.ldw + kb0 + 8 * g;
  h8 xs[kD][4], ws0[kD][4], ws1[kD][4];
  auto load = [&](auto slot, int i) {
    constexpr int s = decltype(slot)::value;
    const size_t off = (size_t)(wave + 4 * i) * kSK;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      load16(xs[s][q], xr + off + 32 * q);
      load16(ws0[s][q], w0 + off + 32 * q);
      load16(ws1[s][q], w1 + off + 32 * q);
    }
  };
  f4 acc0 = f4{0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  auto comp = [&](auto slot) {
    constexpr int s = decltype(slot)::value;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc0 = mfma16(xs[s][q], ws0[s][q], acc0);
      acc1 = mfma16(xs[s][q], ws1[s][q], acc1);
    }
  };
  sfor<0, kD>([&](auto sc) {
    if (decltype(sc)::value < nbw) load(sc, decltype(sc)::value);
  });
  int i = 0;
  for (; i + kD <= nbw; i += kD) {
    sfor<0, kD>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      comp(sc);
      if (i + s + kD < nbw) load(sc, i + s + kD);
    });
  }
  sfor<0, kD>([&](auto sc) {
    if (i + decltype(sc)::value < nbw) comp(sc);
  });

  red[wave][0][lane] = acc0;
  red[wave][1][lane] = acc1;
  __syncthreads();
  if (wave != 0) return;
  f4 s0 = red[0][0][lane], s1 = red[0][1][lane];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    s0 += red[w][0][lane];
    s1 += red[w][1][lane];
  }
  // lane (r, g) holds rows 4 g + e of columns n0 + r (s0) and n0 + 16 + r (s1)
  const uint32_t ca = n0 + r, cbn = n0 + 16 + r;
  if (a.splits > 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t m = 4 * g + e;
      if (m >= M) break;
      float* dst = a.ws + ((size_t)split * M + m) * N;
      if (ca < N) dst[ca] = s0[e];
      if (cbn < N) dst[cbn] = s1[e];
    }
    return;
  }
  const uint32_t epi = mb.epi, ldy = mb.ldy;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t m = 4 * g + e;
    if (m >= M) break;
    if (epi == 3u) {  // SwiGLU: columns n0 .. + 16 are the gate block, n0 + 16 .. + 16 the up block
      if (ca < N) ((_Float16*)mb.y)[(size_t)m * ldy + n0 / 2 + r] = (_Float16)swiglu_f(s0[e], s1[e]);
    } else if (epi == 1u) {
      _Float16* y = (_Float16*)mb.y + (size_t)m * ldy;
      if (ca < N) y[ca] = (_Float16)s0[e];
      if (cbn < N) y[cbn] = (_Float16)s1[e];
    } else {
      float* y = (float*)mb.y + (size_t)m * ldy;
      if (epi == 2u) {
        if (ca < N) y[ca] += s0[e];
        if (cbn < N) y[cbn] += s1[e];
      } else {
        if (ca < N) y[ca] = s0[e];
        if (cbn < N) y[cbn] = s1[e];
      }
    }
  }
}

hipError_t launch_stream(const TileArgs& a, uint32_t grid, hipStream_t s) {
  hipLaunchKernelGGL(gemm_stream_kernel, dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dh
