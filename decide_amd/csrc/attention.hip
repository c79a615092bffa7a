// Causal GQA attention with the sigmoid output gate, for gfx950 MFMA
// (decide: kernels/attn_fast.metal; cpu_ref.rs:167-188):
//   y[r, h·256 + d] = (softmax_j(q_r,h · k_j,h/4 / 16) · v_·,h/4)[d] · σ(gate[r, h·256 + d]),
// over cache rows j = 0 ..= qpos[r]; q, K, V fp16, scores and softmax fp32,
// the softmax weights rounded to fp16 once as the P·V operand, y fp16.
//
// Design (MI355X's own):
//   * A workgroup is one kv head × 32 query rows; its 8 waves are the 4 query
//     heads sharing that kv head × 2 blocks of 16 rows, so one staged K/V tile
//     serves all eight (the tiles come from L2 once per 32 rows, which is what
//     bounds this kernel). The next block's K/V rows are loaded into registers
//     while the current block computes.
//   * Everything is computed transposed: Sᵀ = K·Qᵀ (A = K rows from LDS,
//     B = the wave's Q rows held in registers for the whole kernel) and
//     Oᵀ += Vᵀ·Pᵀ. In the MFMA output layout a lane then holds 8 scores of
//     ONE query row for keys {4g..4g+3, 16+4g..16+4g+3} (g = lane / 16), which
//     is exactly the B operand Pᵀ needs if the 32 keys of a block are taken
//     in that order — so P goes from scores to MFMA operand without leaving
//     registers. Vᵀ is staged key-contiguous (transposed on the way into LDS)
//     and read in the same key order.
//   * Online softmax in the exp2 domain; a row's max is reduced across the
//     four lane groups that hold it; the running sum stays
//     per lane and is reduced once at the end (both reductions by cross-row
//     lane swaps). The reference point moves (and
//     O is rescaled) only when a score passes it by more than 2^8, which after
//     the first blocks almost never happens. Blocks wholly before every row of
//     the wave skip the causal mask.
//   * Query blocks run longest-first so the causal triangle's tail is not
//     the last work scheduled. Rows past `rows` are clamped for loads and
//     skipped for stores; keys past the block's last position are masked
//     (their staged rows are clamped reads of valid cache rows).
#include <type_traits>

#include "dh_kernels.h"

namespace dh {

namespace {
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kHD = 256, kNQ = 16, kQDim = kNQ * kHD;
constexpr int kBQ = 32;    // query rows per workgroup (2 blocks of 16)
constexpr int kBKey = 32;  // keys per block
constexpr int kKLD = kHD + 8;  // K tile row stride (halves): 528 B, conflict-free 16-lane reads
constexpr int kVLD = kBKey + 4;  // Vᵀ tile row stride (halves): 72 B = 18 banks, so 16 rows hit distinct bank pairs
constexpr float kScaleLog2 = 0.0625f * 1.4426950408889634f;  // 1/16 · log2(e)
constexpr float kNeg = -1e30f;
constexpr float kLazy = 8.0f;  // log2 headroom of the softmax reference point (weights up to 256)

// The four lane groups g = lane / 16 that hold one query row, combined with
// gfx950's cross-row swaps (no LDS round trip, unlike a general shuffle):
// permlane16_swap pairs rows 0-1 and 2-3 of 16 lanes, permlane32_swap the two
// halves; called with the same value twice, the two results are x and its
// partner.
__device__ __forceinline__ float max4_rows(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4_rows(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ f4 mfma16(const h8& a, const h8& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
}  // namespace

__global__ __launch_bounds__(512) void attention_kernel(const _Float16* __restrict__ q, const _Float16* __restrict__ kc,
                                                        const _Float16* __restrict__ vc, const float* __restrict__ pq,
                                                        const uint32_t* __restrict__ qpos, _Float16* __restrict__ y,
                                                        uint32_t ldq, uint32_t rows) {
  __shared__ __attribute__((aligned(16))) _Float16 ks[kBKey * kKLD];
  __shared__ __attribute__((aligned(16))) _Float16 vts[kHD * kVLD];
  __shared__ uint32_t wpmax[8];
  const uint32_t qb = gridDim.x - 1 - blockIdx.x;
  const uint32_t kvh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t h = kvh * 4 + (wave & 3);
  const int rl = lane & 15, g = lane >> 4;
  const uint32_t r0 = qb * kBQ + 16 * (wave >> 2);
  const uint32_t row = min(r0 + rl, rows - 1);
  const uint32_t mypos = qpos[row];
  uint32_t pmax = mypos, wminpos = mypos;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    pmax = max(pmax, (uint32_t)__shfl_xor((int)pmax, o, 64));
    wminpos = min(wminpos, (uint32_t)__shfl_xor((int)wminpos, o, 64));
  }
  if (lane == 0) wpmax[wave] = pmax;

  h8 qf[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) qf[c] = *(const h8*)(q + ((size_t)row * kNQ + h) * kHD + 32 * c + 8 * g);
  f4 oacc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) oacc[i] = f4{0.f, 0.f, 0.f, 0.f};
  float m = kNeg, lsum = 0.f;
  __syncthreads();
  // the workgroup's last key: the largest position over its 32 rows (loads past it are clamped to it)
  uint32_t kmax = wpmax[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) kmax = max(kmax, wpmax[i]);

  const uint32_t nblk = kmax / kBKey + 1;
  // staging: K rows as 16-byte chunks (thread → key id / 32, chunk id % 32, two per thread);
  // V as key pairs × 8-dim chunks, transposed into vts on the way in
  const int kp = tid & 15, dc = tid >> 4;
  // two register slots of staged rows: block b + 2 is fetched while block b computes, so a fetch has two
  // blocks' work to land (one block's was not enough: the L2 round trip outlasts it)
  h8 kpre[2][2], vpre[2][2];
  auto fetch = [&](uint32_t kb0, auto sc) {
    constexpr int sl = decltype(sc)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = tid + 512 * i, key = id >> 5, c16 = id & 31;
      kpre[sl][i] = *(const h8*)(kc + ((size_t)min(kb0 + key, kmax) * 4 + kvh) * kHD + 8 * c16);
      vpre[sl][i] = *(const h8*)(vc + ((size_t)min(kb0 + 2 * kp + i, kmax) * 4 + kvh) * kHD + 8 * dc);
    }
  };
  auto block = [&](uint32_t blk, auto sc) {
    constexpr int sl = decltype(sc)::value;
    const uint32_t kb0 = blk * kBKey;
    __syncthreads();  // the previous block's LDS reads are done
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = tid + 512 * i, key = id >> 5, c16 = id & 31;
      *(h8*)(ks + key * kKLD + 8 * c16) = kpre[sl][i];
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) *(h2*)(vts + (8 * dc + d) * kVLD + 2 * kp) = h2{vpre[sl][0][d], vpre[sl][1][d]};
    __syncthreads();
    fetch(kb0 + 2 * kBKey, sc);  // in flight during this block and the next (rows past kmax are clamped reads)

    f4 st[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < 8; ++c) st[kt] = mfma16(*(const h8*)(ks + (16 * kt + rl) * kKLD + 32 * c + 8 * g), qf[c], st[kt]);

    float sv[8];
    if (kb0 + kBKey - 1 <= wminpos) {  // every key of the block is visible to every row of the wave
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = st[i / 4][i % 4] * kScaleLog2;
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t key = kb0 + 16 * kt + 4 * g + e;
          sv[4 * kt + e] = key <= mypos ? st[kt][e] * kScaleLog2 : kNeg;
        }
    }
    float bm = sv[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) bm = fmaxf(bm, sv[i]);
    bm = max4_rows(bm);
    // Lazy rescale: the reference point m moves only when a score exceeds it by more than 2^kLazy, so
    // the weights stay <= 2^kLazy (well inside fp16) and O and the sum are rescaled only on the rare
    // block that moves it (the normalisation uses the same m, so the result does not depend on when).
    if (__any(bm > m + kLazy)) {
      const float mnew = bm > m + kLazy ? bm : m;
      const float alpha = exp2f(m - mnew);
      lsum *= alpha;
      m = mnew;
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[i] *= alpha;
    }
    h8 pb;
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pv = exp2f(sv[i] - m);
      ps += pv;
      pb[i] = (_Float16)pv;
    }
    lsum += ps;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const _Float16* vr = vts + (16 * dt + rl) * kVLD + 4 * g;
      const h4 lo = *(const h4*)vr, hi = *(const h4*)(vr + 16);
      const h8 va = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      oacc[dt] = mfma16(va, pb, oacc[dt]);
    }
  };
  // Blocks in pairs, with no condition inside the pair, so the compiler's wait counts stay exact (a
  // branch there makes it wait for every load at the loop head). A block past the last one (odd nblk)
  // stages clamped rows whose keys are all masked: its scores are -inf, its weights 0 and alpha 1,
  // so it changes nothing.
  fetch(0, std::integral_constant<int, 0>{});
  fetch(kBKey, std::integral_constant<int, 1>{});
  for (uint32_t blk = 0; blk < nblk; blk += 2) {
    block(blk, std::integral_constant<int, 0>{});
    block(blk + 1, std::integral_constant<int, 1>{});
  }

  const float l = sum4_rows(lsum);
  const float inv = 1.0f / l;
  if (r0 + rl < rows) {
    const uint32_t r = r0 + rl;
    const float* gp = pq + (size_t)r * ldq + kQDim + h * kHD;
    _Float16* yp = y + (size_t)r * kQDim + h * kHD;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const int d0 = 16 * dt + 4 * g;
      // gate as two float2 and y as two half2: 8- and 4-byte alignment suffice (decide's contract)
      const f2 g01 = *(const f2*)(gp + d0), g23 = *(const f2*)(gp + d0 + 2);
      const float gt[4] = {g01[0], g01[1], g23[0], g23[1]};
      _Float16 o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (_Float16)(oacc[dt][e] * inv * (1.0f / (1.0f + __expf(-gt[e]))));
      *(h2*)(yp + d0) = h2{o[0], o[1]};
      *(h2*)(yp + d0 + 2) = h2{o[2], o[3]};
    }
  }
}

hipError_t launch_attention(const _Float16* q, const _Float16* kc, const _Float16* vc, const float* pq,
                            const uint32_t* qpos, _Float16* y, uint32_t rows, uint32_t ldq, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(attention_kernel, dim3((rows + kBQ - 1) / kBQ, 4), dim3(512), 0, s, q, kc, vc, pq, qpos, y, ldq,
                     rows);
  return hipGetLastError();
}

}  // namespace dh
