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
//     registers. Vᵀ is transposed on the way into LDS with its keys in that
//     same order, so each lane reads its 8 keys of a Vᵀ row with one
//     16-byte LDS read.
//   * Online softmax in the exp2 domain; a row's max is reduced across the
//     four lane groups that hold it; the running sum stays
//     per lane and is reduced once at the end (both reductions by cross-row
//     lane swaps). The reference point moves (and
//     O is rescaled) only when a score passes it by more than 2^8, which after
//     the first blocks almost never happens. Blocks wholly before every row of
//     the wave skip the causal mask.
//   * One workgroup per CU (two waves per SIMD), so a causal prompt's longest
//     query block (all of its keys) would set the kernel's time while most
//     CUs sit idle. A query block's keys are therefore cut into pieces of L
//     key blocks at fixed offsets (piece p covers blocks [pL, pL + L), the
//     last piece the rest), one workgroup each, dispatched longest-first;
//     a query block with more than one piece writes each piece's (max,
//     sum, unnormalised O) per row and head, and attention_combine_kernel
//     merges them. The cut points depend only on L (chosen on the host from
//     the row count and the key bound), never on the neighbouring rows, so a
//     row whose keys end before a cut gets bit for bit the one-piece result.
//   * Rows past `rows` are clamped for loads and skipped for stores; keys past
//     the block's last position are masked (their staged rows are clamped
//     reads of valid cache rows).
#include <algorithm>
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
// Vᵀ tile row stride (halves): 80 B = 20 banks, 16-byte aligned, so 16 rows' ds_read_b128 hit distinct bank quads
constexpr int kVLD = kBKey + 8;
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

// The largest position over query block qb's 32 rows (rows past `rows` clamped
// to the last one): its last key, the same in both kernels.
__device__ __forceinline__ uint32_t block_kmax(const uint32_t* __restrict__ qpos, uint32_t qb, uint32_t rows,
                                               uint32_t lane) {
  uint32_t v = qpos[min(qb * kBQ + (lane & 31), rows - 1)];
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}

// Pieces query block qb really has: ceil(nblk / L), at most np (the last one
// takes the remainder).
__device__ __forceinline__ uint32_t block_pieces(uint32_t nblk, uint32_t L, uint32_t np) {
  return min(np, (nblk + L - 1) / L);
}

__global__ __launch_bounds__(512) void attention_kernel(const _Float16* __restrict__ q, const _Float16* __restrict__ kc,
                                                        const _Float16* __restrict__ vc, const float* __restrict__ pq,
                                                        const uint32_t* __restrict__ qpos, _Float16* __restrict__ y,
                                                        float* __restrict__ part, uint32_t ldq, uint32_t rows,
                                                        uint32_t L, uint32_t np) {
  __shared__ __attribute__((aligned(16))) _Float16 ks[kBKey * kKLD];
  __shared__ __attribute__((aligned(16))) _Float16 vts[kHD * kVLD];
  __shared__ uint32_t wpmax[8];
  // Work item: kv head fastest, then query blocks longest (last) first, then pieces. The hardware deals
  // workgroups round-robin over the 8 XCDs, so each XCD gets every 8th item: with pieces outermost, any 8
  // consecutive items are two query blocks' worth of the same piece, of about the same length.
  const uint32_t nqb = (rows + kBQ - 1) / kBQ;
  const uint32_t kvh = blockIdx.x & 3;
  const uint32_t qb = nqb - 1 - (blockIdx.x >> 2) % nqb;
  const uint32_t piece = (blockIdx.x >> 2) / nqb;
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
  const uint32_t npieces = block_pieces(nblk, L, np);
  if (piece >= npieces) return;  // uniform over the workgroup: every wave read the same kmax
  // this piece's key blocks: L of them (L even, so the pair loop below covers them exactly), the last piece the
  // rest (its pair loop may run one block past nblk, which is wholly masked)
  const uint32_t b0 = piece * L;
  const uint32_t b1 = piece + 1 == npieces ? nblk : b0 + L;
  // staging: K rows as 16-byte chunks (thread → key id / 32, chunk id % 32, two per thread);
  // V as key pairs × 8-dim chunks, transposed into vts on the way in
  const int kp = tid & 15, dc = tid >> 4;
  // Vᵀ keys are stored in the order the P operand takes them: lane group g's keys {4g..4g+3, 16+4g..16+4g+3} at
  // 8g .. 8g+7, so each lane reads its 8 keys with one ds_read_b128. Key pair (2 kp, 2 kp + 1) lands at vpos.
  const int vpos = ((kp >> 1 & 3) << 3) + ((kp >> 3) << 2) + ((kp & 1) << 1);
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
    for (int d = 0; d < 8; ++d) *(h2*)(vts + (8 * dc + d) * kVLD + vpos) = h2{vpre[sl][0][d], vpre[sl][1][d]};
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
      const h8 va = *(const h8*)(vts + (16 * dt + rl) * kVLD + 8 * g);
      oacc[dt] = mfma16(va, pb, oacc[dt]);
    }
  };
  // Blocks in pairs, with no condition inside the pair, so the compiler's wait counts stay exact (a
  // branch there makes it wait for every load at the loop head). A block past the last one (odd nblk)
  // stages clamped rows whose keys are all masked: its scores are -inf, its weights 0 and alpha 1,
  // so it changes nothing.
  fetch(b0 * kBKey, std::integral_constant<int, 0>{});
  fetch((b0 + 1) * kBKey, std::integral_constant<int, 1>{});
  for (uint32_t blk = b0; blk < b1; blk += 2) {
    block(blk, std::integral_constant<int, 0>{});
    block(blk + 1, std::integral_constant<int, 1>{});
  }

  const float l = sum4_rows(lsum);
  if (npieces > 1) {
    // This piece's state for the combine: O unnormalised (relative to m), and (m, l), where a row with no key in
    // the piece (position before its first key) has weights of exp2(0) on masked scores: its l is written as 0
    // and the combine skips the piece for that row by the same position test.
    if (r0 + rl < rows) {
      const uint32_t prow = nqb * kBQ;
      const size_t slot = ((size_t)piece * prow + r0 + rl) * kNQ + h;
      float* op = part + slot * kHD;
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) *(f4*)(op + 16 * dt + 4 * g) = oacc[dt];
      if (g == 0) {
        float* ml = part + (size_t)np * prow * kNQ * kHD + 2 * slot;
        *(f2*)ml = f2{m, (uint64_t)mypos >= (uint64_t)b0 * kBKey ? l : 0.0f};
      }
    }
    return;
  }
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

// Merges the pieces of every query block that has more than one: a workgroup
// per row, a lane per (query head, 16 dims). Only the pieces whose first key
// the row can see take part (the attention kernel's position test); with one
// such piece the arithmetic is the one-piece path's own (weight exp2(0) = 1),
// so the result is identical.
__global__ __launch_bounds__(256) void attention_combine_kernel(const float* __restrict__ part,
                                                                const float* __restrict__ pq,
                                                                const uint32_t* __restrict__ qpos,
                                                                _Float16* __restrict__ y, uint32_t ldq, uint32_t rows,
                                                                uint32_t L, uint32_t np) {
  const uint32_t r = blockIdx.x, qb = r / kBQ;
  const int tid = threadIdx.x;
  const uint32_t kmax = block_kmax(qpos, qb, rows, tid & 63);
  const uint32_t npieces = block_pieces(kmax / kBKey + 1, L, np);
  if (npieces <= 1) return;  // written by the attention kernel itself
  const uint32_t mypos = qpos[r];
  const uint32_t nv = (uint32_t)min((uint64_t)npieces, (uint64_t)mypos / ((uint64_t)L * kBKey) + 1);
  const uint32_t h = tid >> 4, d0 = 16 * (tid & 15);
  const uint32_t prow = (rows + kBQ - 1) / kBQ * kBQ;
  const size_t pstride = (size_t)prow * kNQ;  // (row, head) slots per piece
  const size_t slot0 = (size_t)r * kNQ + h;
  const float* ml = part + (size_t)np * pstride * kHD;
  float mv[kAttnMaxPieces], lv[kAttnMaxPieces];
#pragma unroll
  for (uint32_t p = 0; p < kAttnMaxPieces; ++p)
    if (p < nv) {
      const f2 st = *(const f2*)(ml + 2 * (p * pstride + slot0));
      mv[p] = st[0];
      lv[p] = st[1];
    }
  float mx = mv[0];
#pragma unroll
  for (uint32_t p = 1; p < kAttnMaxPieces; ++p)
    if (p < nv) mx = fmaxf(mx, mv[p]);
  f4 o[4];
  float l;
  {  // piece 0 holds every row's first key
    const float w = exp2f(mv[0] - mx);
    const f4* op = (const f4*)(part + slot0 * kHD + d0);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = op[j] * w;
    l = lv[0] * w;
  }
#pragma unroll
  for (uint32_t p = 1; p < kAttnMaxPieces; ++p)
    if (p < nv) {
      const float w = exp2f(mv[p] - mx);
      const f4* op = (const f4*)(part + (p * pstride + slot0) * kHD + d0);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] += op[j] * w;
      l += lv[p] * w;
    }
  const float inv = 1.0f / l;
  const float* gp = pq + (size_t)r * ldq + kQDim + h * kHD + d0;
  _Float16* yp = y + (size_t)r * kQDim + h * kHD + d0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const f2 gt = *(const f2*)(gp + 2 * j);
    const float o0 = o[j / 2][2 * (j % 2)], o1 = o[j / 2][2 * (j % 2) + 1];
    *(h2*)(yp + 2 * j) = h2{(_Float16)(o0 * inv * (1.0f / (1.0f + __expf(-gt[0])))),
                            (_Float16)(o1 * inv * (1.0f / (1.0f + __expf(-gt[1]))))};
  }
}

AttnSplit attention_split(uint32_t rows, uint32_t npos, uint32_t cus) {
  AttnSplit sp;
  if (rows == 0) return sp;
  npos = std::max(npos, rows);
  const uint32_t nqb = (rows + kBQ - 1) / kBQ;
  const uint32_t nbm = (npos + kBKey - 1) / kBKey;  // key blocks of the furthest row
  // key blocks over every query block if the rows sit at positions npos - rows .. npos - 1 (a prompt chunk)
  uint64_t est = 0;
  for (uint32_t qb = 0; qb < nqb; ++qb) {
    const uint64_t last = std::min<uint64_t>(npos - 1, (uint64_t)(npos - rows) + (uint64_t)qb * kBQ + kBQ - 1);
    est += last / kBKey + 1;
  }
  // Pieces of 1.3x one CU's even share of the work (4 kv heads), even length, at most kAttnMaxPieceRows / 32
  // query-block pieces in all (the workspace bound). Measured at 2,307 causal rows: 1.0x (L = 44 blocks)
  // 125 us, 1.3x (L = 56) 113 us, 1.5x (L = 64) 122 us; at 1,024 rows 1.3x is also the fastest. Fewer, longer
  // pieces write fewer partial states for the combine; shorter ones balance the CUs better.
  auto even_up = [](uint64_t v) { return (uint32_t)std::max<uint64_t>(2, (v + 1) & ~1ull); };
  const uint32_t cap = std::min<uint32_t>(kAttnMaxPieces, std::max<uint32_t>(1, kAttnMaxPieceRows / kBQ / nqb));
  uint32_t L = even_up((est * 4 * 13 / 10 + cus - 1) / std::max(1u, cus));
  uint32_t np = (nbm + L - 1) / L;
  if (np > cap) {
    L = even_up((nbm + cap - 1) / cap);
    np = (nbm + L - 1) / L;
  }
  if (np <= 1) return sp;
  sp.L = L;
  sp.np = np;
  return sp;
}

uint64_t attention_ws_bytes(uint32_t rows, const AttnSplit& sp) {
  if (sp.np <= 1) return 0;
  const uint64_t prow = (uint64_t)(rows + kBQ - 1) / kBQ * kBQ;
  return (uint64_t)sp.np * prow * kNQ * (kHD + 2) * sizeof(float);
}

uint64_t attention_ws_max(uint32_t max_rows) {
  uint64_t most = 0;
  for (uint32_t nqb = 1; nqb <= (std::max(1u, max_rows) + kBQ - 1) / kBQ; ++nqb) {
    AttnSplit sp;
    sp.np = std::min<uint32_t>(kAttnMaxPieces, std::max<uint32_t>(1, kAttnMaxPieceRows / kBQ / nqb));
    most = std::max(most, attention_ws_bytes(nqb * kBQ, sp));
  }
  return most;
}

hipError_t launch_attention(const _Float16* q, const _Float16* kc, const _Float16* vc, const float* pq,
                            const uint32_t* qpos, _Float16* y, float* part, uint32_t rows, uint32_t ldq,
                            const AttnSplit& sp, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (sp.np == 0 || sp.L == 0 || sp.L % 2 != 0 || (sp.np > 1 && !part)) return hipErrorInvalidValue;
  const uint32_t nqb = (rows + kBQ - 1) / kBQ;
  hipLaunchKernelGGL(attention_kernel, dim3(nqb * sp.np * 4), dim3(512), 0, s, q, kc, vc, pq, qpos, y, part, ldq,
                     rows, sp.L, sp.np);
  if (sp.np > 1) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(rows), dim3(256), 0, s, part, pq, qpos, y, ldq, rows, sp.L,
                       sp.np);
  }
  return hipGetLastError();
}

}  // namespace dh
