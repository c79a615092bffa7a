// MFMA tile GEMM for gfx950: Y = epi(X · Wᵀ), X fp16 [M, K], W fp16 [N, K]
// (both K-contiguous, decide's NT layout), fp32 accumulation.
//
// Role in decide: the `gemm_nt_fast*` tile kernels and, with FM = 1, the
// small-M weight-streaming kernel `gemm_nt_small`
// (kernels/gemm_fast.metal:240-351, 429-566). The design is MI355X's own:
//
//   * Workgroup = WN wavefronts (64 lanes) side by side along N. Every wave
//     computes all BM = 16·FM rows of the tile for its own 16·FN columns with
//     v_mfma_f32_16x16x32_f16, so the X tile is the only operand the waves
//     share: it is staged through LDS, double-buffered (one barrier per stage).
//   * W is used by exactly one wave per workgroup, so it never touches LDS:
//     each lane loads its MFMA B operands straight from global memory into
//     VGPRs, PD stages (of 64 K) ahead of use, 16-byte loads, every 128-byte
//     row segment read whole by four lanes. This is the weight-streaming form;
//     at skinny M it is what keeps HBM busy.
//   * K order inside a stage: sub-step s (0, 1) covers k0 + 32s .. +32, and
//     lane group g = lane / 16 supplies k0 + 32s + 8g .. +8 for both operands,
//     so A and B always pair the same k.
//   * M tail in-kernel: rows past M re-read row M-1 (never stored). N tail:
//     columns past N re-read row N-1 of W (never stored).
//   * Workgroup ids are renumbered so that the consecutive work items of one
//     XCD (the hardware deals workgroups round-robin over the 8 XCDs) walk the
//     M tiles of one W column stripe back to back: the stripe is fetched from
//     HBM once and re-read from that XCD's L2.
//   * Epilogues (decide's four, gemm.rs:15-26) straight from the accumulator
//     registers; SwiGLU pairs fragment j (gate) with j + 1 (up), the
//     16-column blocks of the gate|up interleave.
//   * Split-K: workgroups of split s write fp32 partials; a second kernel sums
//     them in split order (deterministic) and applies the epilogue.
#include "dh_kernels.h"

namespace dh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + __expf(-v)); }

// Workgroup b runs on XCD b % 8. Renumber so XCD x owns one contiguous range
// of work ids (a bijection on [0, G)).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t G) {
  const uint32_t xcd = b & 7u, local = b >> 3;
  const uint32_t per = G >> 3, rem = G & 7u;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

template <int FM, int FN, int WN, int PD>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WN, 64 * WN), amdgpu_waves_per_eu(1, 1)))
void gemm_tile_kernel(const TileArgs p) {
  constexpr int BM = 16 * FM, BN = 16 * FN * WN, NT = 64 * WN;
  constexpr int LDA = kBK + 8;  // LDS row stride in halves (16-byte pad)
  // The X tile is copied by every thread alike: XPT 16-byte chunks each, so
  // the LDS tile has XR >= BM rows (rows past BM are loaded, never read).
  constexpr int RPP = NT / (kBK / 8);  // rows one pass of the workgroup copies
  constexpr int XR = (BM + RPP - 1) / RPP * RPP;
  constexpr int XPT = XR / RPP;
  constexpr int TILE = XR * LDA;  // halves per LDS buffer
  static_assert(FN % 2 == 0, "SwiGLU pairs fragments j, j+1: FN must be even");
  __shared__ __attribute__((aligned(16))) _Float16 lds[2 * TILE];

  // ---- work item of this workgroup
  const uint32_t wid = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t mt = wid % p.mtiles;
  const uint32_t q = wid / p.mtiles;
  const uint32_t split = q % p.splits;
  const uint32_t gs = q / p.splits;
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxMembers; ++i)
    if (i < (int)p.count && gs >= p.mem[i].stripe_begin) mi = i;
  const _Float16* __restrict__ W = p.mem[mi].w;
  const uint32_t ldw = p.mem[mi].ldw, N = p.mem[mi].n;
  const uint32_t M = p.m;
  const uint32_t m0 = mt * BM;
  const uint32_t n0 = (gs - p.mem[mi].stripe_begin) * BN;
  const uint32_t kb = split * p.kps;
  const uint32_t ke = min(p.k, kb + p.kps);
  const int nst = (int)((ke - kb) / kBK);  // full 64-wide stages
  const bool half_tail = ((ke - kb) % kBK) != 0;  // one more 32-wide sub-stage

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;

  // ---- X (A operand) chunk addresses of this thread: rows xrow0 + c·RPP,
  // 16-byte column xcol of the 128-byte stage row.
  const int xrow0 = tid / (kBK / 8), xcol = tid % (kBK / 8);
  const _Float16* xp[XPT];
#pragma unroll
  for (int c = 0; c < XPT; ++c) {
    const uint32_t grow = min(m0 + (uint32_t)(xrow0 + c * RPP), M - 1);
    xp[c] = p.x + (size_t)grow * p.ldx + kb + xcol * 8;
  }
  const int xl0 = xrow0 * LDA + xcol * 8;  // LDS offset of chunk 0; chunk c adds c·RPP·LDA
  // ---- W (B operand) row addresses of this lane: fragment j covers columns
  // n0 + wave·16·FN + 16 j .. + 16; this lane feeds column (… + r).
  const _Float16* wp[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const uint32_t n = min(n0 + (uint32_t)(wave * 16 * FN + j * 16 + r), N - 1);
    wp[j] = W + (size_t)n * ldw + kb + g * 8;
  }

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  h8 wr[PD][FN][2];
  u4 xr[XPT];

  auto load_w = [&](h8 (&dst)[FN][2], int kt) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int s = 0; s < 2; ++s) dst[j][s] = *(const h8*)(wp[j] + kt * kBK + s * 32);
  };
  auto load_x = [&](int kt) {
#pragma unroll
    for (int c = 0; c < XPT; ++c) xr[c] = *(const u4*)(xp[c] + kt * kBK);
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int c = 0; c < XPT; ++c) *(u4*)(lds + buf * TILE + xl0 + c * RPP * LDA) = xr[c];
  };

  // ---- prologue
#pragma unroll
  for (int pp = 0; pp < PD; ++pp)
    if (pp < nst) load_w(wr[pp], pp);
  if (nst > 0) {
    load_x(0);
    store_x(0);
  }
  __syncthreads();

  // ---- one pipeline stage: X(kt + 1) global → registers, the 2·FM·FN MFMAs
  // of stage kt, W(kt + PD) → the ring slot just consumed, X(kt + 1) → LDS.
  auto stage = [&](int kt, h8 (&wbuf)[FN][2], bool prefetch, bool more) {
    if (more) load_x(kt + 1);
    // Keep the X loads ahead of the MFMAs: they have one stage to land.
    __builtin_amdgcn_sched_barrier(0);
    const _Float16* A = lds + (kt & 1) * TILE;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const h8 a = *(const h8*)(A + (i * 16 + r) * LDA + s * 32 + g * 8);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, wbuf[j][s], acc[i][j], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (prefetch) load_w(wbuf, kt + PD);
    if (more) store_x((kt + 1) & 1);
    __syncthreads();
  };

  // ---- steady state: groups of PD stages that all prefetch, with no
  // conditions inside, so the compiler's load counters stay exact.
  int kt = 0;
  for (; kt + 2 * PD <= nst; kt += PD) {
#pragma unroll
    for (int pp = 0; pp < PD; ++pp) stage(kt + pp, wr[pp], true, true);
  }
  // ---- drain: the last < 2·PD stages (kt is a multiple of PD here)
#pragma unroll
  for (int pp = 0; pp < 2 * PD; ++pp) {
    if (kt + pp < nst) stage(kt + pp, wr[pp % PD], kt + pp + PD < nst, kt + pp + 1 < nst);
  }

  // ---- K % 64 == 32: one last 32-wide sub-stage, not pipelined
  if (half_tail) {
    const int kt = nst;
    h8 wt[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) wt[j] = *(const h8*)(wp[j] + kt * kBK);
    if (xcol < 4) {  // the first 32 halves of each row only
#pragma unroll
      for (int c = 0; c < XPT; ++c) *(u4*)(lds + xl0 + c * RPP * LDA) = *(const u4*)(xp[c] + kt * kBK);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const h8 a = *(const h8*)(lds + (i * 16 + r) * LDA + g * 8);
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, wt[j], acc[i][j], 0, 0, 0);
    }
  }

  // ---- epilogue. Accumulator element e of fragment (i, j) in lane (r, g) is
  // row m0 + 16 i + 4 g + e, column nw + 16 j + r.
  const uint32_t nw = n0 + wave * 16 * FN;
  if (p.splits > 1) {
    float* ws = p.ws + (size_t)split * M * N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t row = m0 + i * 16 + g * 4 + e;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const uint32_t col = nw + j * 16 + r;
          if (col < N) ws[(size_t)row * N + col] = acc[i][j][e];
        }
      }
    return;
  }
  const uint32_t epi = p.mem[mi].epi, ldy = p.mem[mi].ldy;
  void* Y = p.mem[mi].y;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t row = m0 + i * 16 + g * 4 + e;
      if (row >= M) continue;
      const size_t rb = (size_t)row * ldy;
      if (epi == 3u) {
#pragma unroll
        for (int j = 0; j < FN; j += 2) {
          const uint32_t col = nw + j * 16 + r;
          if (col >= N) continue;
          const float o = silu_f(acc[i][j][e]) * acc[i][j + 1][e];
          ((_Float16*)Y)[rb + (nw + j * 16) / 2 + r] = (_Float16)o;
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const uint32_t col = nw + j * 16 + r;
          if (col >= N) continue;
          const float v = acc[i][j][e];
          if (epi == 0u)
            ((float*)Y)[rb + col] = v;
          else if (epi == 1u)
            ((_Float16*)Y)[rb + col] = (_Float16)v;
          else
            ((float*)Y)[rb + col] += v;
        }
      }
    }
}

// ---- the compiled menu. (FM, FN, WN, PD)
#define DH_TILE_MENU(X) \
  X(1, 2, 4, 4)         \
  X(2, 2, 4, 4)         \
  X(4, 2, 4, 3)         \
  X(4, 4, 4, 3)         \
  X(6, 4, 4, 2)         \
  X(8, 4, 4, 2)         \
  X(10, 4, 4, 2)        \
  X(12, 4, 4, 2)        \
  X(13, 4, 4, 2)        \
  X(14, 4, 4, 2)        \
  X(15, 4, 4, 2)        \
  X(16, 4, 4, 2)        \
  X(8, 2, 4, 2)         \
  X(13, 2, 4, 2)

struct VariantEntry {
  VariantInfo info;
  void (*fn)(const TileArgs);
};

#define DH_TILE_ENTRY(FM, FN, WN, PD) {{FM, FN, WN}, gemm_tile_kernel<FM, FN, WN, PD>},
static const VariantEntry kVariants[] = {DH_TILE_MENU(DH_TILE_ENTRY)};
#undef DH_TILE_ENTRY

int variant_count() { return (int)(sizeof(kVariants) / sizeof(kVariants[0])); }
VariantInfo variant_info(int v) { return kVariants[v].info; }

hipError_t launch_tile(int v, const TileArgs& a, uint32_t grid, hipStream_t s) {
  const VariantEntry& e = kVariants[v];
  hipLaunchKernelGGL(e.fn, dim3(grid), dim3(64 * e.info.wn), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Split-K reduction: y = epi(Σ_s ws[s]) summed in split order. One thread per
// output element (SwiGLU: per fp16 output, reading its gate and up sums).
__global__ void splitk_reduce_kernel(const float* __restrict__ ws, uint32_t splits, uint32_t m, uint32_t n, void* y,
                                     uint32_t ldy, uint32_t epi) {
  const uint32_t ncols = epi == 3u ? n / 2 : n;
  const size_t total = (size_t)m * ncols;
  const size_t plane = (size_t)m * n;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(t / ncols), oc = (uint32_t)(t % ncols);
    if (epi == 3u) {
      const uint32_t gc = (oc / kSwigluBlock) * 2 * kSwigluBlock + oc % kSwigluBlock;
      const float* pg = ws + (size_t)row * n + gc;
      float gsum = 0.f, usum = 0.f;
      for (uint32_t s = 0; s < splits; ++s) {
        gsum += pg[s * plane];
        usum += pg[s * plane + kSwigluBlock];
      }
      ((_Float16*)y)[(size_t)row * ldy + oc] = (_Float16)(silu_f(gsum) * usum);
    } else {
      const float* pp = ws + (size_t)row * n + oc;
      float v = 0.f;
      for (uint32_t s = 0; s < splits; ++s) v += pp[s * plane];
      const size_t o = (size_t)row * ldy + oc;
      if (epi == 0u)
        ((float*)y)[o] = v;
      else if (epi == 1u)
        ((_Float16*)y)[o] = (_Float16)v;
      else
        ((float*)y)[o] += v;
    }
  }
}

hipError_t launch_splitk_reduce(const float* ws, uint32_t splits, uint32_t m, uint32_t n, void* y, uint32_t ldy,
                                uint32_t epi, hipStream_t s) {
  const size_t total = (size_t)m * (epi == 3u ? n / 2 : n);
  const uint32_t blocks = (uint32_t)std::min<size_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, ws, splits, m, n, y, ldy, epi);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Reference kernel (DH_GEMM_REFERENCE): one output per thread, fp32 FMA over K
// in order, so every row is computed the same way whatever M is. The analog
// of decide's baseline `gemm_nt` (kernels/gemm.metal:13-76), used to bisect.
__global__ void gemm_reference_kernel(const _Float16* __restrict__ x, uint32_t ldx, const _Float16* __restrict__ w,
                                      uint32_t ldw, void* y, uint32_t ldy, uint32_t m, uint32_t n, uint32_t k,
                                      uint32_t epi) {
  const uint32_t ncols = epi == 3u ? n / 2 : n;
  const uint32_t oc = blockIdx.x * blockDim.x + threadIdx.x;
  if (oc >= ncols) return;
  for (uint32_t row = blockIdx.y; row < m; row += gridDim.y) {
  const _Float16* xr = x + (size_t)row * ldx;
  auto dot = [&](uint32_t col) {
    const _Float16* wr = w + (size_t)col * ldw;
    float a = 0.f;
    for (uint32_t kk = 0; kk < k; ++kk) a = fmaf((float)xr[kk], (float)wr[kk], a);
    return a;
  };
  const size_t o = (size_t)row * ldy + oc;
  if (epi == 3u) {
    const uint32_t gc = (oc / kSwigluBlock) * 2 * kSwigluBlock + oc % kSwigluBlock;
    ((_Float16*)y)[o] = (_Float16)(silu_f(dot(gc)) * dot(gc + kSwigluBlock));
  } else {
    const float v = dot(oc);
    if (epi == 0u)
      ((float*)y)[o] = v;
    else if (epi == 1u)
      ((_Float16*)y)[o] = (_Float16)v;
    else
      ((float*)y)[o] += v;
  }
  }
}

hipError_t launch_gemm_reference(const _Float16* x, uint32_t ldx, const _Float16* w, uint32_t ldw, void* y,
                                 uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi, hipStream_t s) {
  const uint32_t ncols = epi == 3u ? n / 2 : n;
  hipLaunchKernelGGL(gemm_reference_kernel, dim3((ncols + 127) / 128, std::min<uint32_t>(m, 4096)), dim3(128), 0, s, x, ldx, w, ldw, y, ldy, m,
                     n, k, epi);
  return hipGetLastError();
}

}  // namespace dh
