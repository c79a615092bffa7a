// MFMA tile GEMM for gfx950: Y = epi(X · Wᵀ), X fp16 [M, K], W fp16 [N, K]
// (both K-contiguous, decide's NT layout), fp32 accumulation.
//
// Role in decide: the `gemm_nt_fast*` tile kernels and, with FM <= 2, the
// small-M weight-streaming kernel `gemm_nt_small`
// (kernels/gemm_fast.metal:240-351, 429-566). The design is MI355X's own:
//
//   * Workgroup = 4 wavefronts side by side along N, 64 columns each, every
//     wave computing all BM = 16·FM rows of the tile with
//     v_mfma_f32_16x16x32_f16 (BN = 256). The 2 x 2 variants arrange the
//     4 waves 2 x 2 with FM x FN fragments each (32·FM x 32·FN tiles): each
//     wave reads only half of the tile's X rows and half of its W rows from
//     LDS, so LDS bytes per output fall with the tile's area; 160 x 288 makes
//     exactly one gate|up tile per CU at M ≈ 603.
//   * Both operands reach LDS by coalesced DMA (global_load_lds_dwordx4:
//     eight lanes per 128-byte row segment, no VGPR staging). The MFMA B
//     operand wants 16 different W rows per load instruction; gathered
//     straight from L2 that pattern runs at well under half the bandwidth of
//     the coalesced DMA, so W goes through LDS too.
//   * LDS rows are 128 bytes (one 64-wide K stage), unpadded; the 16-byte
//     chunk c of row rr is stored at chunk c ^ ((rr >> 1) & 7): every DMA
//     instruction writes 1 KB contiguously and the ds_read_b128 of 16
//     consecutive rows spreads over all banks.
//   * Rings of NBX X-tile and NBW W-tile stage buffers (W, the operand that
//     streams from HBM, gets the deeper one; small tiles, whose stages are
//     short, take 5-deep rings so a DMA has several stages to land). The
//     DMAs the next stage needs are issued at the start of a stage, the rest
//     are spread over its MFMAs; one vmcnt wait and one barrier per stage.
//   * LDS reads just in time (stage_s): per k-half, the operand with fewer
//     fragments per wave is read whole, the other streamed one fragment per
//     group of MFMAs, a few groups ahead; the stage's barrier comes before its
//     last groups, which run from registers while the next stage's first
//     reads are in flight (tiles with too few fragments per half keep the
//     read-everything-first schedule, stage()).
//   * The hot loop (LDS reads, MFMAs, waits, DMAs) is inline asm in program
//     order: accumulators pinned in AGPRs so the register allocator cannot
//     rotate them, and exact wait counts.
//   * K order inside a stage: sub-step s (0, 1) covers k0 + 32s .. +32, and
//     lane group g = lane / 16 supplies k0 + 32s + 8g .. +8 for both operands.
//   * M tail in-kernel: rows past M re-read row M-1 (never stored). N tail:
//     columns past N re-read row N-1 of W (never stored). K % 64 == 32: one
//     unpipelined 32-wide sub-stage at the end.
//   * Workgroup ids are renumbered so that the consecutive work items of one
//     XCD (the hardware deals workgroups round-robin over the 8 XCDs) walk the
//     M tiles of one W column stripe back to back: the stripe is fetched from
//     HBM once and re-read from that XCD's L2.
//   * Epilogues (decide's four, gemm.rs:15-26) through LDS so every wave
//     writes whole output rows with 16-byte stores; SwiGLU pairs fragment j
//     (gate) with j + 1 (up), the 16-column blocks of the gate|up interleave.
//   * Split-K: workgroups of split s write fp32 partials; a second kernel sums
//     them in split order (deterministic) and applies the epilogue.
#include "tile_common.h"

namespace dh {

// Epilogue through LDS for the 4-wave tiles (WM waves along M, 4 / WM along
// N, each wave FM x FN fragments): the accumulators of CR = 64 rows at a time
// are written to LDS in row-major fp32 (row stride BN + 4 floats: the four
// lane groups of a store land 16 banks apart), then read back so that each
// wave writes whole output rows with 16-byte stores. `stage` must hold
// 64 · (BN + 4) floats and be free (all main-loop LDS reads done).
template <int FM, int FN, int WM>
__device__ __forceinline__ void store_tile_lds(f4 (&acc)[FM][FN], const TileArgs& p, int mi, uint32_t split,
                                               uint32_t m0, uint32_t n0, int wave, int r, int g, float* stage) {
  constexpr int WN = 4 / WM, BN = 16 * FN * WN, LDR = BN + 4, CR = 64, BM = 16 * FM * WM;
  static_assert(WM == 1 || FN % 2 == 1, "2 x 2 layouts: SwiGLU handles one straddling pair (odd fragments per wave)");
  const int rbase = (wave / WN) * 16 * FM, cbase = (wave % WN) * 16 * FN;  // this wave's sub-tile
  const uint32_t M = p.m, N = p.mem[mi].n;
  const int tid = threadIdx.x;
  const uint32_t epi = p.mem[mi].epi, ldy = p.mem[mi].ldy;
  char* Y = (char*)p.mem[mi].y;
  const bool partial = p.splits > 1;
  const uint32_t esz = (partial || epi == 0u || epi == 2u) ? 4u : 2u;
  const bool vec16 = partial || ((((uintptr_t)Y) % 16) == 0 && ((size_t)ldy * esz) % 16 == 0);
  if constexpr (WM == 1) {
  if (epi == 3u && !partial) {
    // SwiGLU in registers (a wave holds whole gate|up pairs), then the fp16
    // tile [BM][BN/2] through LDS (row stride BN + 16 bytes) and out with
    // 16-byte stores, 16 lanes per row.
    constexpr int OW = BN / 2;          // output halves per tile row
    constexpr int LDH = OW + 8;         // LDS row stride in halves
    _Float16* st = (_Float16*)stage;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; j += 2) {
        pin_acc(acc[i][j]);
        pin_acc(acc[i][j + 1]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          st[(i * 16 + 4 * g + e) * LDH + wave * 8 * FN + (j / 2) * 16 + r] =
              (_Float16)swiglu_f(acc[i][j][e], acc[i][j + 1][e]);
      }
    __syncthreads();
    constexpr int OQ = OW / 8;  // 16-byte chunks per row
#pragma unroll
    for (int it = 0; it < (BM * OQ + 255) / 256; ++it) {
      const int item = it * 256 + tid;
      if (item >= BM * OQ) break;
      const int row = item / OQ, oq = item % OQ;
      const uint32_t grow = m0 + row;
      if (grow >= M || n0 + 32 * (oq / 2) >= N) continue;
      const h8 o = *(const h8*)(st + row * LDH + oq * 8);
      _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + (n0 / 2) + oq * 8;
      if (vec16) {
        __builtin_nontemporal_store(o, (h8*)dst);  // streamed out: nothing re-reads it in this kernel
      } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int q = 0; q < 8; q += 2) *(h2*)(dst + q) = h2{o[q], o[q + 1]};
      }
    }
    return;
  }
  } else if constexpr (FN % 2 == 1) {
  if (epi == 3u && !partial) {
    // 2 x 2 waves with an odd fragment count per wave: each wave holds 4 of
    // its gate|up pairs whole (SwiGLU in registers, as above) and one half of
    // the pair that straddles the two N halves, which goes through LDS in
    // fp32 (gate from the left waves, up from the right ones).
    constexpr int OW = BN / 2, LDH = OW + 8, PS = (FN - 1) / 2;  // PS: the straddling pair
    _Float16* st = (_Float16*)stage;
    float* gsp = (float*)(st + BM * LDH);  // [BM][16] gate, then [BM][16] up
    float* usp = gsp + BM * 16;
    __syncthreads();
    // WNC: this wave's N half (compile time, so every accumulator index is a constant)
    auto pairs = [&](auto wnc) {
      constexpr int WNC = decltype(wnc)::value, J0 = WNC;  // local fragment J0 starts the first whole pair
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        static_for<0, (FN - J0) / 2>([&](auto qc) {
          constexpr int j = J0 + 2 * decltype(qc)::value;  // local pair (j, j + 1)
          constexpr int col = ((WNC * FN + j) / 2) * 16;
          pin_acc(acc[i][j]);
          pin_acc(acc[i][j + 1]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            st[(rbase + i * 16 + 4 * g + e) * LDH + col + r] = (_Float16)swiglu_f(acc[i][j][e], acc[i][j + 1][e]);
        });
        pin_acc(acc[i][WNC == 0 ? FN - 1 : 0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (WNC == 0)
            gsp[(rbase + i * 16 + 4 * g + e) * 16 + r] = acc[i][FN - 1][e];
          else
            usp[(rbase + i * 16 + 4 * g + e) * 16 + r] = acc[i][0][e];
        }
      }
    };
    if (wave % WN == 0)
      pairs(std::integral_constant<int, 0>{});
    else
      pairs(std::integral_constant<int, 1>{});
    __syncthreads();
#pragma unroll
    for (int it = 0; it < (BM * 16 + 255) / 256; ++it) {
      const int item = it * 256 + tid;
      if (item >= BM * 16) break;
      st[(item / 16) * LDH + PS * 16 + item % 16] = (_Float16)swiglu_f(gsp[item], usp[item]);
    }
    __syncthreads();
    constexpr int OQ = OW / 8;  // 16-byte chunks per row
#pragma unroll
    for (int it = 0; it < (BM * OQ + 255) / 256; ++it) {
      const int item = it * 256 + tid;
      if (item >= BM * OQ) break;
      const int row = item / OQ, oq = item % OQ;
      const uint32_t grow = m0 + row;
      if (grow >= M || n0 + 32 * (oq / 2) >= N) continue;
      const h8 o = *(const h8*)(st + row * LDH + oq * 8);
      _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + (n0 / 2) + oq * 8;
      if (vec16) {
        __builtin_nontemporal_store(o, (h8*)dst);
      } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int q = 0; q < 8; q += 2) *(h2*)(dst + q) = h2{o[q], o[q + 1]};
      }
    }
    return;
  }
  }
  static_for<0, (BM + CR - 1) / CR>([&](auto cc) {
    constexpr int c0 = decltype(cc)::value * CR;
    constexpr int rows = (BM - c0) < CR ? (BM - c0) : CR;
    if (m0 + c0 >= M) return;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int tr = rbase + 16 * i;  // fragments never straddle a CR boundary
      if (tr < c0 || tr >= c0 + CR) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        pin_acc(acc[i][j]);
#pragma unroll
        for (int e = 0; e < 4; ++e) stage[(tr - c0 + 4 * g + e) * LDR + cbase + j * 16 + r] = acc[i][j][e];
      }
    }
    __syncthreads();
    // SwiGLU reaches this path only as split-K partials (raw fp32; the reduce applies it).
    // One float4 of a tile row per item.
#pragma unroll
    for (int it = 0; it < (rows * (BN / 4) + 255) / 256; ++it) {
      const int item = it * 256 + tid;
      if (item >= rows * (BN / 4)) break;
      const int row = item / (BN / 4), cq = item % (BN / 4);
      const uint32_t grow = m0 + c0 + row, gcol = n0 + 4 * cq;
      if (grow >= M || gcol >= N) continue;
      const f4 v = *(const f4*)(stage + row * LDR + 4 * cq);
      if (partial) {
        __builtin_nontemporal_store(v, (f4*)(p.ws + ((size_t)split * M + grow) * N + gcol));
      } else if (epi == 1u) {
        _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + gcol;
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        *(h2*)dst = h2{(_Float16)v[0], (_Float16)v[1]};
        *(h2*)(dst + 2) = h2{(_Float16)v[2], (_Float16)v[3]};
      } else {
        float* dst = (float*)Y + (size_t)grow * ldy + gcol;
        typedef float fl2 __attribute__((ext_vector_type(2)));
        if (vec16) {
          f4 o = v;
          if (epi == 2u) o += *(const f4*)dst;
          *(f4*)dst = o;
        } else {
          fl2 lo = fl2{v[0], v[1]}, hi = fl2{v[2], v[3]};
          if (epi == 2u) {
            lo += *(const fl2*)dst;
            hi += *(const fl2*)(dst + 2);
          }
          *(fl2*)dst = lo;
          *(fl2*)(dst + 2) = hi;
        }
      }
    }
  });
}

// Epilogue of the 2 x 2 tiles with swapped MFMA operands (Pipe<..., SW>): lane (r, g) of a wave holds, for
// fragment (i, j), row 16i + r and columns 16j + 4g .. +3 of the wave's block, so every output leaves straight
// from registers: fp32 / fp16 / split-K partials as 16- or 8-byte stores of 4 consecutive columns, SwiGLU as
// 8-byte stores of 4 outputs from a whole gate|up pair. Only the pair that straddles the two N halves (FN odd:
// the left waves hold its gate, the right waves its up) passes through LDS, in fp32. The values stored are
// those of store_tile_lds, bit for bit.
template <int FM, int FN>
__device__ __forceinline__ void store_tile_sw(f4 (&acc)[FM][FN], const TileArgs& p, int mi, uint32_t split,
                                              uint32_t m0, uint32_t n0, int wave, int r, int g, float* stage) {
  static_assert(FN % 2 == 1, "2 x 2 layouts: SwiGLU handles one straddling pair (odd fragments per wave)");
  constexpr int WN = 2;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  typedef float fl2 __attribute__((ext_vector_type(2)));
  const int wm = wave / WN, wn = wave % WN, lane = r + 16 * g;
  const uint32_t rbase = (uint32_t)(wm * 16 * FM), cbase = (uint32_t)(wn * 16 * FN);
  const uint32_t M = p.m, N = p.mem[mi].n;
  const uint32_t epi = p.mem[mi].epi, ldy = p.mem[mi].ldy;
  char* Y = (char*)p.mem[mi].y;
  const bool partial = p.splits > 1;
  if (epi == 3u && !partial) {
    const bool v8 = (((uintptr_t)Y) % 8) == 0 && ((size_t)ldy * 2) % 8 == 0;
    // four outputs silu(g)·u of one row at output column ocol (a multiple of 4)
    auto put = [&](uint32_t grow, uint32_t ocol, const f4& gv, const f4& uv) {
      h4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (_Float16)swiglu_f(gv[e], uv[e]);
      _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + ocol;
      if (v8) {
        *(h4*)dst = o;  // a quarter line per 16 lanes: plain stores, so L2 merges the lines before HBM
      } else {
        *(h2*)dst = h2{o[0], o[1]};
        *(h2*)(dst + 2) = h2{o[2], o[3]};
      }
    };
    f4* xch = (f4*)stage + wm * FM * 64;  // the straddling pair's gate, [FM][64 lanes] per M half
    __syncthreads();                      // every wave is past its last read of the main loop's LDS
    if (wn == 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        pin_acc(acc[i][FN - 1]);
        xch[i * 64 + lane] = acc[i][FN - 1];
      }
    }
    auto pairs = [&](auto wnc) {
      constexpr int J0 = decltype(wnc)::value;  // the first local fragment that starts a whole pair
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const uint32_t grow = m0 + rbase + 16 * i + r;
        static_for<0, (FN - J0) / 2>([&](auto qc) {
          constexpr int j = J0 + 2 * decltype(qc)::value;
          pin_acc(acc[i][j]);
          pin_acc(acc[i][j + 1]);
          const uint32_t gcol = n0 + cbase + 16 * j;  // the pair's gate block, a multiple of 32
          if (grow < M && gcol < N) put(grow, gcol / 2 + 4 * g, acc[i][j], acc[i][j + 1]);
        });
      }
    };
    if (wn == 0)
      pairs(std::integral_constant<int, 0>{});
    else
      pairs(std::integral_constant<int, 1>{});
    __syncthreads();
    if (wn == 1) {
      const uint32_t gcol = n0 + 16 * (FN - 1);  // the straddling pair's gate block
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const uint32_t grow = m0 + rbase + 16 * i + r;
        pin_acc(acc[i][0]);
        const f4 gv = xch[i * 64 + lane];
        if (grow < M && gcol < N) put(grow, gcol / 2 + 4 * g, gv, acc[i][0]);
      }
    }
    return;
  }
  const uint32_t esz = (partial || epi == 0u || epi == 2u) ? 4u : 2u;
  const bool vec = partial || ((((uintptr_t)Y) % (4 * esz)) == 0 && ((size_t)ldy * esz) % (4 * esz) == 0);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const uint32_t grow = m0 + rbase + 16 * i + r;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      pin_acc(acc[i][j]);
      const uint32_t gcol = n0 + cbase + 16 * j + 4 * g;
      if (grow >= M || gcol >= N) continue;
      const f4 v = acc[i][j];
      if (partial) {
        *(f4*)(p.ws + ((size_t)split * M + grow) * N + gcol) = v;
      } else if (epi == 1u) {
        _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + gcol;
        const h4 o = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        if (vec) {
          *(h4*)dst = o;
        } else {
          *(h2*)dst = h2{o[0], o[1]};
          *(h2*)(dst + 2) = h2{o[2], o[3]};
        }
      } else {
        float* dst = (float*)Y + (size_t)grow * ldy + gcol;
        if (vec) {
          f4 o = v;
          if (epi == 2u) o += *(const f4*)dst;
          *(f4*)dst = o;
        } else {
          fl2 lo = fl2{v[0], v[1]}, hi = fl2{v[2], v[3]};
          if (epi == 2u) {
            lo += *(const fl2*)dst;
            hi += *(const fl2*)(dst + 2);
          }
          *(fl2*)dst = lo;
          *(fl2*)(dst + 2) = hi;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The tile pipeline: NBX X-tile and NBW W-tile stage buffers; stage kt issues
// X(kt + NBX - 1) and W(kt + NBW - 1). The DMAs a stage issues are ordered so
// that the ones needed by the next stage come first; one vmcnt wait then
// covers exactly those.
template <int FM, int FN_, int WM, int NBX, int NBW, bool SW = false>
struct Pipe {
  static constexpr int FN = FN_, WN = 4 / WM, NT = 256, LAX = NBX - 1, LAW = NBW - 1;
  static constexpr int U = (NBX == NBW) ? NBX : NBX * NBW;  // unroll (lcm for 2, 3)
  static constexpr int LAM = LAX > LAW ? LAX : LAW;
  static constexpr int BM = 16 * FM * WM, BN = 16 * FN * WN;
  static constexpr int XR = (BM + 31) / 32 * 32;
  static constexpr int XPW = XR / 32;
  static constexpr int WPW = BN / 32;  // W DMAs per wave per stage (8 rows each)
  static constexpr int XBYTES = XR * 128, WBYTES = BN * 128;
  static constexpr int WRING = NBX * XBYTES;  // offset of the W ring
  static constexpr int LDS_BYTES = NBX * XBYTES + NBW * WBYTES;
  // outstanding DMAs allowed at the end of a stage (those not needed next):
  // with equal depths, the DMAs of stages kt + 2 .. kt + LA
  static constexpr int KEEP = NBX == NBW ? (LAX - 1) * (XPW + WPW) : (LAX >= 2 ? XPW : 0) + (LAW >= 2 ? WPW : 0);
  static_assert(NBX >= 2 && NBW >= 2 && ((NBX == NBW && NBX <= 5) || (NBX == 2 && NBW == 3)),
                "ring depths: equal (2 to 5), or 2 for X and 3 for W");
  static_assert(KEEP + XPW + WPW <= 63, "outstanding DMAs fit the vmcnt counter");
  static_assert((WM == 1 && FN == 4) || WM == 2, "wave layouts: 1 x 4 with 4 fragments per wave, or 2 x 2");
  static_assert(BN % 32 == 0, "whole 8-row DMA groups per wave");

  f4 acc[FM][FN];
  // acc += X fragment · W fragmentᵀ. With SW the MFMA takes W as its A operand, so each accumulator holds its
  // 16 x 16 block transposed (lane (r, g): row r, columns 4g .. 4g+3); swapping the operands leaves every sum
  // bitwise the same.
  __device__ __forceinline__ static void mma(f4& c, const h8& xa, const h8& wb) {
    if constexpr (SW)
      mfma_acc_v(c, wb, xa);
    else
      mfma_acc_v(c, xa, wb);
  }
  uint32_t xoff[XPW];
  uint32_t woff[WPW];
  uint32_t a0, a1;
  uint32_t xrow;  // LDS byte offset of this wave's first X row (its M half)
  uint32_t lds_addr;
  uint32_t xm0[XPW];
  uint32_t wm0;
  uint32_t wrow;
  const char* wbase;
  const char* xbase;

  template <int B>
  __device__ __forceinline__ void dma_x(int kt) {
    const char* xb = xbase + (size_t)kt * (kBK * 2);
#pragma unroll
    for (int q = 0; q < XPW; ++q) dma16(lds_addr + B * XBYTES + xm0[q], xoff[q], xb);
  }
  template <int B>
  __device__ __forceinline__ void dma_w(int kt) {
    const char* wb = wbase + (size_t)kt * (kBK * 2);
#pragma unroll
    for (int q = 0; q < WPW; ++q) dma16(lds_addr + WRING + B * WBYTES + wm0 + q * 1024, woff[q], wb);
  }
  // issue the DMAs of stage kt for the rings (X slot BX, W slot BW), needed-next first
  template <int BX, int BW>
  __device__ __forceinline__ void issue(int kt, int nst) {
    const bool ix = kt + LAX < nst, iw = kt + LAW < nst;
    if (LAX <= LAW) {
      if (ix) dma_x<(BX + LAX) % NBX>(kt + LAX);
      if (iw) dma_w<(BW + LAW) % NBW>(kt + LAW);
    } else {
      if (iw) dma_w<(BW + LAW) % NBW>(kt + LAW);
      if (ix) dma_x<(BX + LAX) % NBX>(kt + LAX);
    }
  }
  template <int F>
  static constexpr int a_imm() {
    return (F % FM) * 16 * 128;
  }
  // One stage's DMA number D (compile time): X blocks first, then W blocks,
  // into ring slots NX / NW, for stages kx / kw.
  template <int D, int NX, int NW>
  __device__ __forceinline__ void dma_one(int kx, int kw) {
    if constexpr (D < XPW) {
      dma16(lds_addr + NX * XBYTES + xm0[D], xoff[D], xbase + (size_t)kx * (kBK * 2));
    } else {
      dma16(lds_addr + WRING + NW * WBYTES + wm0 + (D - XPW) * 1024, woff[D - XPW],
            wbase + (size_t)kw * (kBK * 2));
    }
  }
  // The MFMAs of a stage from ring slots (BX, BW). With IL, the DMAs of stage
  // kt + LAX / kt + LAW are spread over the fragments (one every NF / DPW),
  // so the address unit sees a steady stream instead of a burst that would
  // stall the issuing waves.
  template <int BX, int BW, bool IL, bool XFIRST>
  __device__ __forceinline__ void compute(int kt) {
    constexpr int NF = 2 * FM, AD = 2, DPW = XPW + WPW;
    constexpr int NXS = (BX + LAX) % NBX, NWS = (BW + LAW) % NBW;
    const uint32_t xb = lds_addr + BX * XBYTES;
    const uint32_t b0 = xb + xrow + a0, b1 = xb + xrow + a1;
    const uint32_t wb = lds_addr + WRING + BW * WBYTES + wrow;
    const uint32_t w0 = wb + a0, w1 = wb + a1;
    h8 wf[FN][2];
    static_for<0, FN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      ds_read16<j * 16 * 128>(wf[j][0], w0);
      ds_read16<j * 16 * 128>(wf[j][1], w1);
    });
    h8 a[AD + 1];
    static_for<0, AD>([&](auto fc) {
      constexpr int f = decltype(fc)::value;
      ds_read16<a_imm<f>()>(a[f], f / FM ? b1 : b0);
    });
    static_for<0, NF>([&](auto fc) {
      constexpr int f = decltype(fc)::value;
      if constexpr (IL) {
        // The DMAs the next stage needs (the operand with lookahead 1) go out
        // together before the first fragment; the others (lookahead 2) are
        // spread one every NF / n fragments over the rest of the stage.
        constexpr int NEED = (LAX == 1 ? XPW : 0) + (LAW == 1 ? WPW : 0);
        constexpr int REST = DPW - NEED;
        static_for<0, DPW>([&](auto dc) {
          constexpr int d = decltype(dc)::value;
          constexpr int dd = XFIRST ? d : (d < WPW ? d + XPW : d - WPW);  // issue order
          constexpr int at = d < NEED ? 0 : (REST > 0 ? (d - NEED) * NF / REST : 0);
          if constexpr (at == f) dma_one<dd, NXS, NWS>(kt + LAX, kt + LAW);
        });
      }
      if constexpr (f + AD < NF) ds_read16<a_imm<f + AD>()>(a[(f + AD) % (AD + 1)], (f + AD) / FM ? b1 : b0);
      constexpr int later = (NF - 1 - f) < AD ? (NF - 1 - f) : AD;
      wait_lgkm<later>();
      tie(a[f % (AD + 1)]);
      if constexpr (f == 0) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          tie(wf[j][0]);
          tie(wf[j][1]);
        }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) mma(acc[f % FM][j], a[f % (AD + 1)], wf[j][f / FM]);
    });
  }
  // Stage kt; U-periodic slot indices are compile-time via Q = kt mod U.
  template <int Q>
  __device__ __forceinline__ void stage(int kt, int nst, bool steady) {
    constexpr int BX = Q % NBX, BW = Q % NBW;
    if (steady) {
      compute<BX, BW, true, (LAX <= LAW)>(kt);
    } else {
      issue<BX, BW>(kt, nst);
      compute<BX, BW, false, true>(kt);
    }
    if (kt + 1 < nst) wait_next(kt, nst, steady);
    __syncthreads();
  }
  // Waits until the DMAs stage kt + 1 reads have landed, leaving in flight
  // only this stage's issues that stage kt + 1 does not need.
  __device__ __forceinline__ void wait_next(int kt, int nst, bool steady) {
    if (steady) {
      wait_vm<KEEP>();
    } else if constexpr (NBX == NBW && NBX > 3) {
      // near the end of K: the stages kt + 2 .. kt + LA that exist were issued
      const int later = min(kt + LAX, nst - 1) - (kt + 1);
      static_for<0, LAX>([&](auto cc) {
        constexpr int c = decltype(cc)::value;
        if (later == c) wait_vm<c * (XPW + WPW)>();
      });
    } else {
      const bool ix2 = LAX >= 2 && kt + LAX < nst, iw2 = LAW >= 2 && kt + LAW < nst;
      if (ix2 && iw2)
        wait_vm<XPW + WPW>();
      else if (ix2)
        wait_vm<XPW>();
      else if (iw2)
        wait_vm<WPW>();
      else
        wait_vm<0>();
    }
  }

  // ---- The streamed schedule (stage_s): fragments read just in time. ----
  // Per stage and k-half h, the operand with fewer fragments per wave (R:
  // X when FM <= FN) is read whole and held for the half; the other (S) is
  // streamed, one fragment per group of NR MFMAs (group g = (h, s):
  // acc += R(h, 0..NR-1) x S(h, s)). The stage's LDS reads, in the order the
  // groups need them, are R(0, *), S(0, *), R(1, *), S(1, *); the reads group g
  // needs are issued LAG groups ahead (LAG + 1 in the second half, so that all
  // are out LAG groups before the stage ends). The stage's barrier sits
  // before its last NB groups: every wave has its reads of this stage back by
  // then, so after the barrier the next stage's first reads go out while
  // those last groups run from registers, and the DMAs the next stage issues
  // may overwrite this stage's slots.
  static constexpr bool RA = FM <= FN;
  static constexpr int NR = RA ? FM : FN, NS = RA ? FN : FM;
  static constexpr int NG = 2 * NS, NL = 2 * (NR + NS);
  static constexpr int LAG = 3, NB = 3;
  static constexpr int GB = NG - NB;  // the barrier comes before group GB
  // used when each half has enough groups for the lookahead (else stage())
  static constexpr bool STREAMED = NS > LAG + 1 && GB >= 2;
  // the index (in the stage's read order) of the last read group g needs
  static constexpr int need(int g) { return (g / NS) * (NR + NS) + NR + g % NS; }
  // reads issued once group g has issued its own (all of them by group GB - 1)
  static constexpr int issued(int g) {
    const int la = g < NS ? LAG : LAG + 1;
    return need(g + la < NG - 1 ? g + la : NG - 1) + 1;
  }
  static constexpr int ENTRY = need(LAG - 1) + 1;  // issued before group 0 (by the previous stage)
  static_assert(!STREAMED || issued(GB - 1) == NL, "every read of a stage is issued before its barrier");

  h8 rf[2][NR], sf[2][NS];

  // Read I of the stage whose X and W sit in ring slots BX and BW.
  template <int I, int BX, int BW>
  __device__ __forceinline__ void read_one() {
    constexpr int h = I / (NR + NS), q = I % (NR + NS);
    constexpr bool isr = q < NR;
    constexpr int f = isr ? q : q - NR;
    constexpr bool isx = isr == RA;  // an X (A operand) fragment
    const uint32_t kh = h ? a1 : a0;
    const uint32_t base = isx ? lds_addr + BX * XBYTES + xrow + kh : lds_addr + WRING + BW * WBYTES + wrow + kh;
    if constexpr (isr)
      ds_read16<(isx ? (f % FM) : f) * 16 * 128>(rf[h][f], base);
    else
      ds_read16<(isx ? (f % FM) : f) * 16 * 128>(sf[h][f], base);
  }
  template <int B, int E, int BX, int BW>
  __device__ __forceinline__ void read_range() {
    static_for<B, E>([&](auto ic) { read_one<decltype(ic)::value, BX, BW>(); });
  }
  // The first ENTRY reads of the stage in slots (BX, BW).
  template <int BX, int BW>
  __device__ __forceinline__ void entry_reads() {
    read_range<0, ENTRY, BX, BW>();
  }
  // Stage kt in ring slots (Q mod NBX, Q mod NBW); its first ENTRY reads were
  // issued before it.
  template <int Q>
  __device__ __forceinline__ void stage_s(int kt, int nst, bool steady) {
    constexpr int BX = Q % NBX, BW = Q % NBW;
    constexpr int NX = (Q + 1) % NBX, NW = (Q + 1) % NBW;
    constexpr int NXS = (BX + LAX) % NBX, NWS = (BW + LAW) % NBW;
    constexpr int DPW = XPW + WPW;
    constexpr int NEED = (LAX == 1 ? XPW : 0) + (LAW == 1 ? WPW : 0);  // DMAs stage kt + 1 needs: issued first
    constexpr int REST = DPW - NEED;
    if (!steady) issue<BX, BW>(kt, nst);
    static_for<0, NG>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      constexpr int h = g / NS, s = g % NS;
      if constexpr (g == GB) {
        wait_lgkm<0>();
        if (kt + 1 < nst) wait_next(kt, nst, steady);
        __syncthreads();
        if (kt + 1 < nst) entry_reads<NX, NW>();
      }
      if constexpr (g < GB) {
        // this stage's DMAs for stage kt + LA: the ones stage kt + 1 needs at group 0, the rest spread to GB - 1
        static_for<0, DPW>([&](auto dc) {
          constexpr int d = decltype(dc)::value;
          constexpr int dd = (LAX <= LAW) ? d : (d < WPW ? d + XPW : d - WPW);  // issue order
          constexpr int at = d < NEED ? 0 : 1 + (REST > 0 ? (d - NEED) * (GB - 1) / REST : 0);
          if constexpr (at == g) {
            if (steady) dma_one<dd, NXS, NWS>(kt + LAX, kt + LAW);
          }
        });
        read_range<g == 0 ? ENTRY : issued(g - 1), issued(g), BX, BW>();
        constexpr int pending = issued(g) - need(g) - 1;
        wait_lgkm<(pending < 15 ? pending : 15)>();
        tie(sf[h][s]);
        if constexpr (s == 0) {
#pragma unroll
          for (int r = 0; r < NR; ++r) tie(rf[h][r]);
        }
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if constexpr (RA)
          mma(acc[r][s], rf[h][r], sf[h][s]);
        else
          mma(acc[s][r], sf[h][s], rf[h][r]);
      }
    });
  }
};

// Work id -> (M tile, column stripe, K split). K splits are outermost. Within
// a split, ngroup = 0 runs the M tiles fastest (consecutive ids share a
// stripe's W); ngroup = g runs the stripes in groups of g, each group's stripes
// fastest and then its M tiles, so that the contiguous run of ids one XCD gets
// from xcd_remap covers a block of about (run / g) M tiles by g stripes: the
// XCD's L2 then fetches fewer distinct X rows and W columns (the planner picks
// g, plan.cpp). Every id below mtiles · nstripes · splits maps to a distinct
// in-range triple: grp · g < nstripes, so gsz >= 1.
__device__ __forceinline__ void tile_coords(const TileArgs& p, uint32_t wid, uint32_t& mt, uint32_t& gs,
                                            uint32_t& split) {
  const uint32_t per_split = p.mtiles * p.nstripes;
  split = wid / per_split;
  const uint32_t rem = wid - split * per_split;
  if (p.ngroup == 0) {
    mt = rem % p.mtiles;
    gs = rem / p.mtiles;
    return;
  }
  const uint32_t gw = p.mtiles * p.ngroup;
  const uint32_t grp = rem / gw, local = rem - grp * gw;
  const uint32_t gsz = min(p.ngroup, p.nstripes - grp * p.ngroup);
  mt = local / gsz;
  gs = grp * p.ngroup + local % gsz;
}

// One tile: FM x FN fragments per wave, WM waves along M and 4 / WM along N.
template <int FM, int FN, int WM, int NBX, int NBW, bool SW = false>
__device__ __forceinline__ void tile_body(const TileArgs& p) {
  using P = Pipe<FM, FN, WM, NBX, NBW, SW>;
  constexpr int BN = P::BN;
  constexpr int LDSB = P::LDS_BYTES > 64 * (BN + 4) * 4 ? P::LDS_BYTES : 64 * (BN + 4) * 4;
  __shared__ __attribute__((aligned(1024))) char lds[LDSB];

  uint32_t mt, gs, split;
  tile_coords(p, xcd_remap(blockIdx.x, gridDim.x), mt, gs, split);
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxMembers; ++i)
    if (i < (int)p.count && gs >= p.mem[i].stripe_begin) mi = i;
  const uint32_t ldw = p.mem[mi].ldw, N = p.mem[mi].n, M = p.m;
  const uint32_t m0 = mt * P::BM;
  const uint32_t n0 = (gs - p.mem[mi].stripe_begin) * BN;
  const uint32_t kb = split * p.kps;
  const uint32_t ke = min(p.k, kb + p.kps);
  const int nst = (int)((ke - kb) / kBK);
  const bool half_tail = ((ke - kb) % kBK) != 0;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  P pp;
  pp.lds_addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  pp.wbase = (const char*)(p.mem[mi].w + kb);
  pp.xbase = (const char*)(p.x + kb);
  const uint32_t sw = (uint32_t)((r >> 1) & 7);
  pp.a0 = r * 128 + ((g ^ sw) * 16);
  pp.a1 = r * 128 + (((4 + g) ^ sw) * 16);
#pragma unroll
  for (int c = 0; c < P::XPW; ++c) {
    const int G = 4 * c + wave;
    const uint32_t row = 8 * G + (lane >> 3);
    const uint32_t chunk = (uint32_t)((lane & 7) ^ ((4 * G + (lane >> 4)) & 7));
    pp.xoff[c] = (min(m0 + row, M - 1) * p.ldx + chunk * 8) * 2;
    pp.xm0[c] = (uint32_t)G * 1024;
  }
#pragma unroll
  for (int c = 0; c < P::WPW; ++c) {
    const int G = P::WPW * wave + c;
    const uint32_t row = 8 * G + (lane >> 3);
    const uint32_t chunk = (uint32_t)((lane & 7) ^ ((4 * G + (lane >> 4)) & 7));
    pp.woff[c] = (min(n0 + row, N - 1) * ldw + chunk * 8) * 2;
  }
  pp.wm0 = (uint32_t)(wave * P::WPW) * 1024;
  pp.wrow = (uint32_t)((wave % P::WN) * 16 * FN) * 128;
  pp.xrow = (uint32_t)((wave / P::WN) * 16 * FM) * 128;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) pp.acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  if (nst > 0) {
    // prologue: X(0..LAX-1) and W(0..LAW-1) in flight; stage 0's land first.
    pp.template dma_x<0>(0);
    pp.template dma_w<0>(0);
    if constexpr (NBX == NBW && NBX > 3) {
      static_for<1, P::LAX>([&](auto sc) {
        constexpr int st = decltype(sc)::value;
        if (st < nst) {
          pp.template dma_x<st>(st);
          pp.template dma_w<st>(st);
        }
      });
      const int later = min(P::LAX, nst) - 1;  // stages issued after stage 0
      static_for<0, P::LAX>([&](auto cc) {
        constexpr int c = decltype(cc)::value;
        if (later == c) wait_vm<c * (P::XPW + P::WPW)>();
      });
    } else {
      int later = 0;  // DMAs issued after stage 0's
      if (nst > 1) {
        if (P::LAX >= 2) {
          pp.template dma_x<1 % NBX>(1);
          later += P::XPW;
        }
        if (P::LAW >= 2) {
          pp.template dma_w<1 % NBW>(1);
          later += P::WPW;
        }
      }
      if (later == P::XPW + P::WPW)
        wait_vm<P::XPW + P::WPW>();
      else if (later == P::XPW)
        wait_vm<P::XPW>();
      else if (later == P::WPW)
        wait_vm<P::WPW>();
      else
        wait_vm<0>();
    }
    __syncthreads();
    if constexpr (P::STREAMED) pp.template entry_reads<0, 0>();

    int kt = 0;
    for (; kt + P::U - 1 + P::LAM < nst; kt += P::U) {
      static_for<0, P::U>([&](auto qc) {
        constexpr int qq = decltype(qc)::value;
        if constexpr (P::STREAMED)
          pp.template stage_s<qq>(kt + qq, nst, true);
        else
          pp.template stage<qq>(kt + qq, nst, true);
      });
    }
    static_for<0, P::U + P::LAM>([&](auto qc) {
      constexpr int qq = decltype(qc)::value;
      if (kt + qq < nst) {
        if constexpr (P::STREAMED)
          pp.template stage_s<qq % P::U>(kt + qq, nst, false);
        else
          pp.template stage<qq % P::U>(kt + qq, nst, false);
      }
    });
  }

  if (half_tail) {  // K % 64 == 32: one 32-wide sub-stage into slot 0, unpipelined
    const char* xb = pp.xbase + (size_t)nst * (kBK * 2);
    const char* wb = pp.wbase + (size_t)nst * (kBK * 2);
#pragma unroll
    for (int c = 0; c < P::XPW; ++c) {
      const int G = 4 * c + wave;
      const uint32_t chunk = (uint32_t)((lane & 7) ^ ((4 * G + (lane >> 4)) & 7));
      if (chunk < 4) dma16(pp.lds_addr + pp.xm0[c], pp.xoff[c], xb);
    }
#pragma unroll
    for (int c = 0; c < P::WPW; ++c) {
      const int G = P::WPW * wave + c;
      const uint32_t chunk = (uint32_t)((lane & 7) ^ ((4 * G + (lane >> 4)) & 7));
      if (chunk < 4) dma16(pp.lds_addr + P::WRING + pp.wm0 + c * 1024, pp.woff[c], wb);
    }
    wait_vm<0>();
    __syncthreads();
    const uint32_t b0 = pp.lds_addr + pp.xrow + pp.a0;
    const uint32_t w0 = pp.lds_addr + P::WRING + pp.wrow + pp.a0;
    h8 wf[FN];
    static_for<0, FN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      ds_read16<j * 16 * 128>(wf[j], w0);
    });
    static_for<0, FM>([&](auto fc) {
      constexpr int i = decltype(fc)::value;
      h8 a;
      ds_read16<i * 16 * 128>(a, b0);
      wait_lgkm<0>();
      tie(a);
      if constexpr (i == 0) {
#pragma unroll
        for (int j = 0; j < FN; ++j) tie(wf[j]);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) P::mma(pp.acc[i][j], a, wf[j]);
    });
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  if constexpr (SW)
    store_tile_sw<FM, FN>(pp.acc, p, mi, split, m0, n0, wave, r, g, (float*)lds);
  else
    store_tile_lds<FM, FN, WM>(pp.acc, p, mi, split, m0, n0, wave, r, g, (float*)lds);
}

template <int FM, int NBX, int NBW>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_tile_kernel(const TileArgs p) {
  tile_body<FM, 4, 1, NBX, NBW>(p);
}

// 2 x 2 waves, each FM x FN fragments: BM = 32·FM, BN = 32·FN. A gate|up
// pair may straddle the two N halves, so SwiGLU runs from the staged tile.
template <int FM, int FN, int NBX, int NBW, bool SW = false>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_tile22_kernel(const TileArgs p) {
  tile_body<FM, FN, 2, NBX, NBW, SW>(p);
}
// ---------------------------------------------------------------------------
// 8-wave BM x BN tiles, two waves per SIMD (BM = 32·FM, BN = 32·(FNA + FNB)). A wave
// reads LDS at about 32 bytes per clock however many reads it keeps in
// flight, so four waves draw at most ~128 B/clk from a CU's LDS, which serves
// about twice that to eight; and eight waves store an epilogue with twice the
// threads. The 2 x 2 tile's quadrants (BM/2 x BN/2) are each split between the
// two waves of one SIMD: BM/2 x 16·FNA ("wide", waves 0-3) and BM/2 x 16·FNB
// ("narrow", waves 4-7); wave w runs on SIMD w % 4 and takes quadrant
// (w % 4 / 2, w % 2). Every output still gets its MFMAs in the same K order
// as in Pipe, so these tiles store the same bits as the other variants.
// A stage's DMAs (BM/8 X row groups of 8 rows, then BN/8 W groups) go to the
// waves round-robin: DMA D belongs to wave D % 8. With 256 x 256 the two rings
// (X 2 deep, W 3 deep) fill the whole 160 KB of LDS.
// DMAs of each kind that wave w (of 8) issues per stage, for NG groups starting at group B
constexpr int t8_count(int w, int B, int NG) {
  int c = 0;
  for (int D = w; D < B + NG; D += 8) c += D >= B;
  return c;
}

template <int FM_, int FN, int XPW, int WPW, int BN>
struct Pipe8 {
  static constexpr int FM = FM_, NBX = 2, NBW = 3, LAX = 1, LAW = 2, U = 6;
  static constexpr int XBYTES = 32 * FM * 128, WBYTES = BN * 128, WRING = NBX * XBYTES;
  static constexpr int LDS_BYTES = NBX * XBYTES + NBW * WBYTES;
  static constexpr int DPW = XPW + WPW;
  static constexpr int KEEP = WPW;  // at a stage's end: stage kt + 2's W DMAs stay in flight
  static_assert(XPW >= 1 && WPW >= 1 && KEEP + DPW <= 63, "DMAs per wave");

  f4 acc[FM][FN];
  uint32_t doff[DPW];  // per-lane source byte offsets (X row groups, then W row groups)
  uint32_t dlds[DPW];  // LDS byte offset of each group inside its ring slot (wave-uniform)
  uint32_t a0, a1, xrow, wrow, lds_addr;
  const char* wbase;
  const char* xbase;

  template <int D, int NX, int NW>
  __device__ __forceinline__ void dma_one(int kx, int kw) {
    if constexpr (D < XPW)
      dma16(lds_addr + NX * XBYTES + dlds[D], doff[D], xbase + (size_t)kx * (kBK * 2));
    else
      dma16(lds_addr + WRING + NW * WBYTES + dlds[D], doff[D], wbase + (size_t)kw * (kBK * 2));
  }
  template <int B>
  __device__ __forceinline__ void dma_x(int kt) {
    static_for<0, XPW>([&](auto dc) { dma_one<decltype(dc)::value, B, 0>(kt, 0); });
  }
  template <int B>
  __device__ __forceinline__ void dma_w(int kt) {
    static_for<XPW, DPW>([&](auto dc) { dma_one<decltype(dc)::value, 0, B>(0, kt); });
  }
  template <int BX, int BW>
  __device__ __forceinline__ void issue(int kt, int nst) {
    if (kt + LAX < nst) dma_x<(BX + LAX) % NBX>(kt + LAX);
    if (kt + LAW < nst) dma_w<(BW + LAW) % NBW>(kt + LAW);
  }
  __device__ __forceinline__ void wait_next(int kt, int nst, bool steady) {
    if (steady || kt + LAW < nst)
      wait_vm<KEEP>();
    else
      wait_vm<0>();
  }

  // The streamed schedule of Pipe::stage_s, for this wave's FM x FN block.
  static constexpr bool RA = FM <= FN;
  static constexpr int NR = RA ? FM : FN, NS = RA ? FN : FM;
  static constexpr int NG = 2 * NS, NL = 2 * (NR + NS);
  static constexpr int LAG = 3, NB = 3, GB = NG - NB;
  static constexpr int need(int g) { return (g / NS) * (NR + NS) + NR + g % NS; }
  static constexpr int issued(int g) {
    const int la = g < NS ? LAG : LAG + 1;
    return need(g + la < NG - 1 ? g + la : NG - 1) + 1;
  }
  static constexpr int ENTRY = need(LAG - 1) + 1;
  static_assert(NS > LAG + 1 && GB >= 2 && issued(GB - 1) == NL, "streamed schedule");

  h8 rf[2][NR], sf[2][NS];

  template <int I, int BX, int BW>
  __device__ __forceinline__ void read_one() {
    constexpr int h = I / (NR + NS), q = I % (NR + NS);
    constexpr bool isr = q < NR;
    constexpr int f = isr ? q : q - NR;
    constexpr bool isx = isr == RA;
    const uint32_t kh = h ? a1 : a0;
    const uint32_t base = isx ? lds_addr + BX * XBYTES + xrow + kh : lds_addr + WRING + BW * WBYTES + wrow + kh;
    if constexpr (isr)
      ds_read16<f * 16 * 128>(rf[h][f], base);
    else
      ds_read16<f * 16 * 128>(sf[h][f], base);
  }
  template <int B, int E, int BX, int BW>
  __device__ __forceinline__ void read_range() {
    static_for<B, E>([&](auto ic) { read_one<decltype(ic)::value, BX, BW>(); });
  }
  template <int BX, int BW>
  __device__ __forceinline__ void entry_reads() {
    read_range<0, ENTRY, BX, BW>();
  }
  template <int Q>
  __device__ __forceinline__ void stage_s(int kt, int nst, bool steady) {
    constexpr int BX = Q % NBX, BW = Q % NBW;
    constexpr int NX = (Q + 1) % NBX, NW = (Q + 1) % NBW;
    constexpr int NXS = (BX + LAX) % NBX, NWS = (BW + LAW) % NBW;
    constexpr int NEED = XPW;  // X (lookahead 1) is needed by stage kt + 1: issued at group 0
    constexpr int REST = DPW - NEED;
    if (!steady) issue<BX, BW>(kt, nst);
    static_for<0, NG>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      constexpr int h = g / NS, s = g % NS;
      if constexpr (g == GB) {
        wait_lgkm<0>();
        if (kt + 1 < nst) wait_next(kt, nst, steady);
        __syncthreads();
        if (kt + 1 < nst) entry_reads<NX, NW>();
      }
      if constexpr (g < GB) {
        static_for<0, DPW>([&](auto dc) {
          constexpr int d = decltype(dc)::value;
          constexpr int at = d < NEED ? 0 : 1 + (d - NEED) * (GB - 1) / REST;
          if constexpr (at == g) {
            if (steady) dma_one<d, NXS, NWS>(kt + LAX, kt + LAW);
          }
        });
        read_range<g == 0 ? ENTRY : issued(g - 1), issued(g), BX, BW>();
        constexpr int pending = issued(g) - need(g) - 1;
        wait_lgkm<(pending < 15 ? pending : 15)>();
        tie(sf[h][s]);
        if constexpr (s == 0) {
#pragma unroll
          for (int r = 0; r < NR; ++r) tie(rf[h][r]);
        }
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if constexpr (RA)
          mfma_acc_v(acc[r][s], rf[h][r], sf[h][s]);
        else
          mfma_acc_v(acc[s][r], sf[h][s], rf[h][r]);
      }
    });
  }
};

// Epilogue of the 8-wave tile, through LDS in fp32 (row stride BN + 4 floats):
// 128 rows at a time, each wave writes its fragments of those rows, then all
// 512 threads store whole rows with 16-byte stores (SwiGLU reads each
// 8-column output chunk's gate and up halves back from the staged rows).
// PAIRS (both halves' fragment counts even, so every wave's first column is
// a multiple of 32 and it holds whole gate|up pairs): SwiGLU runs in
// registers and the fp16 tile goes through LDS once, the same values with a
// quarter of the barriers and half the LDS bytes.
template <int FM, int FN, int BN, bool PAIRS>
__device__ __forceinline__ void store_tile8(f4 (&acc)[FM][FN], const TileArgs& p, int mi, uint32_t split, uint32_t m0,
                                            uint32_t n0, int rbase, int cbase, int r, int g, float* stage) {
  constexpr int LDR = BN + 4, CR = 128, NT = 512, BM = 32 * FM;
  const uint32_t M = p.m, N = p.mem[mi].n;
  const int tid = threadIdx.x;
  const uint32_t epi = p.mem[mi].epi, ldy = p.mem[mi].ldy;
  char* Y = (char*)p.mem[mi].y;
  const bool partial = p.splits > 1;
  const uint32_t esz = (partial || epi == 0u || epi == 2u) ? 4u : 2u;
  const bool vec16 = partial || ((((uintptr_t)Y) % 16) == 0 && ((size_t)ldy * esz) % 16 == 0);
  if constexpr (PAIRS) {
    if (epi == 3u && !partial) {
      constexpr int OW = BN / 2, LDH = OW + 8, OQ = OW / 8;  // fp16 row stride (halves), 16-byte chunks per row
      static_assert(FN % 2 == 0, "whole gate|up pairs per wave");
      _Float16* st = (_Float16*)stage;
      __syncthreads();  // every wave is past its main-loop LDS reads
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; j += 2) {
          pin_acc(acc[i][j]);
          pin_acc(acc[i][j + 1]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            st[(rbase + 16 * i + 4 * g + e) * LDH + cbase / 2 + (j / 2) * 16 + r] =
                (_Float16)swiglu_f(acc[i][j][e], acc[i][j + 1][e]);
        }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < (BM * OQ + NT - 1) / NT; ++it) {
        const int item = it * NT + tid;
        if (item >= BM * OQ) break;
        const int row = item / OQ, oq = item % OQ;
        const uint32_t grow = m0 + row;
        if (grow >= M || n0 + 32 * (oq / 2) >= N) continue;
        const h8 o = *(const h8*)(st + row * LDH + oq * 8);
        _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + (n0 / 2) + oq * 8;
        if (vec16) {
          __builtin_nontemporal_store(o, (h8*)dst);
        } else {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int e = 0; e < 8; e += 2) *(h2*)(dst + e) = h2{o[e], o[e + 1]};
        }
      }
      return;
    }
  }
  static_for<0, (BM + CR - 1) / CR>([&](auto cc) {
    constexpr int c0 = decltype(cc)::value * CR;
    constexpr int rows = (BM - c0) < CR ? (BM - c0) : CR;
    if (m0 + c0 >= M) return;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int tr = rbase + 16 * i;  // fragments never straddle a CR boundary
      if (tr < c0 || tr >= c0 + CR) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        pin_acc(acc[i][j]);
#pragma unroll
        for (int e = 0; e < 4; ++e) stage[(tr - c0 + 4 * g + e) * LDR + cbase + j * 16 + r] = acc[i][j][e];
      }
    }
    __syncthreads();
    if (epi == 3u && !partial) {
      // output chunk q of a row: columns 8q .. 8q + 7 of the fp16 [.., N/2] output
      constexpr int OQ = BN / 16;
#pragma unroll
      for (int it = 0; it < (rows * OQ + NT - 1) / NT; ++it) {
        const int item = it * NT + tid;
        if (item >= rows * OQ) break;
        const int row = item / OQ, q = item % OQ;
        const uint32_t grow = m0 + c0 + row;
        const int gc = 32 * (q / 2) + 8 * (q % 2);
        if (grow >= M || n0 + 32 * (q / 2) >= N) continue;
        const float* sr = stage + row * LDR + gc;
        const f4 g0 = *(const f4*)sr, g1 = *(const f4*)(sr + 4);
        const f4 u0 = *(const f4*)(sr + 16), u1 = *(const f4*)(sr + 20);
        h8 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = (_Float16)swiglu_f(g0[e], u0[e]);
          o[4 + e] = (_Float16)swiglu_f(g1[e], u1[e]);
        }
        _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + (n0 / 2) + 8 * q;
        if (vec16) {
          __builtin_nontemporal_store(o, (h8*)dst);
        } else {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int e = 0; e < 8; e += 2) *(h2*)(dst + e) = h2{o[e], o[e + 1]};
        }
      }
      return;
    }
#pragma unroll
    for (int it = 0; it < (rows * (BN / 4) + NT - 1) / NT; ++it) {
      const int item = it * NT + tid;
      if (item >= rows * (BN / 4)) break;
      const int row = item / (BN / 4), cq = item % (BN / 4);
      const uint32_t grow = m0 + c0 + row, gcol = n0 + 4 * cq;
      if (grow >= M || gcol >= N) continue;
      const f4 v = *(const f4*)(stage + row * LDR + 4 * cq);
      if (partial) {
        __builtin_nontemporal_store(v, (f4*)(p.ws + ((size_t)split * M + grow) * N + gcol));
      } else if (epi == 1u) {
        _Float16* dst = (_Float16*)Y + (size_t)grow * ldy + gcol;
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        *(h2*)dst = h2{(_Float16)v[0], (_Float16)v[1]};
        *(h2*)(dst + 2) = h2{(_Float16)v[2], (_Float16)v[3]};
      } else {
        float* dst = (float*)Y + (size_t)grow * ldy + gcol;
        typedef float fl2 __attribute__((ext_vector_type(2)));
        if (vec16) {
          f4 o = v;
          if (epi == 2u) o += *(const f4*)dst;
          *(f4*)dst = o;
        } else {
          fl2 lo = fl2{v[0], v[1]}, hi = fl2{v[2], v[3]};
          if (epi == 2u) {
            lo += *(const fl2*)dst;
            hi += *(const fl2*)(dst + 2);
          }
          *(fl2*)dst = lo;
          *(fl2*)(dst + 2) = hi;
        }
      }
    }
  });
}

// One wave's share of the 8-wave tile: FN fragments per wave (FNA or FNB), its DMAs per stage.
template <int FM, int FN, int FNA, int FNB, int W0>
__device__ __forceinline__ void tile8_wave(const TileArgs& p, char* lds, int wave, int mi, uint32_t m0, uint32_t n0,
                                           uint32_t split, int nst, bool half_tail, uint32_t ldw, uint32_t N,
                                           uint32_t kb) {
  constexpr int BN = 32 * (FNA + FNB), XG = 4 * FM;  // X row groups of 8 rows
  constexpr int XPW = t8_count(W0, 0, XG), WPW = t8_count(W0, XG, BN / 8);
  static_assert(t8_count(W0, 0, XG) == t8_count(W0 + 3, 0, XG) && t8_count(W0, XG, BN / 8) == t8_count(W0 + 3, XG, BN / 8),
                "the four waves of one path issue the same DMA counts");
  using P = Pipe8<FM, FN, XPW, WPW, BN>;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const uint32_t M = p.m;
  const int simd = wave & 3, mh = simd >> 1, nq = 2 * (simd & 1) + (wave >> 2);
  const int rbase = 16 * FM * mh, cbase = 16 * (FNA + FNB) * (nq >> 1) + 16 * FNA * (nq & 1);
  P pp;
  pp.lds_addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  pp.wbase = (const char*)(p.mem[mi].w + kb);
  pp.xbase = (const char*)(p.x + kb);
  const uint32_t sw = (uint32_t)((r >> 1) & 7);
  pp.a0 = r * 128 + ((g ^ sw) * 16);
  pp.a1 = r * 128 + (((4 + g) ^ sw) * 16);
  pp.xrow = (uint32_t)rbase * 128;
  pp.wrow = (uint32_t)cbase * 128;
#pragma unroll
  for (int d = 0; d < P::DPW; ++d) {
    const int D = wave + 8 * d;                // global DMA index: X groups, then W groups
    const int G = d < XPW ? D : D - XG;        // row group inside its operand
    const uint32_t row = 8 * G + (lane >> 3);  // tile-local row
    const uint32_t chunk = (uint32_t)((lane & 7) ^ ((row >> 1) & 7));
    if (d < XPW)
      pp.doff[d] = (min(m0 + row, M - 1) * p.ldx + chunk * 8) * 2;
    else
      pp.doff[d] = (min(n0 + row, N - 1) * ldw + chunk * 8) * 2;
    pp.dlds[d] = (uint32_t)G * 1024;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) pp.acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  if (nst > 0) {
    pp.template dma_x<0>(0);
    pp.template dma_w<0>(0);
    if (nst > 1) {
      pp.template dma_w<1>(1);
      wait_vm<WPW>();
    } else {
      wait_vm<0>();
    }
    __syncthreads();
    pp.template entry_reads<0, 0>();
    int kt = 0;
    for (; kt + P::U - 1 + P::LAW < nst; kt += P::U) {
      static_for<0, P::U>([&](auto qc) { pp.template stage_s<decltype(qc)::value>(kt + decltype(qc)::value, nst, true); });
    }
    static_for<0, P::U + P::LAW>([&](auto qc) {
      constexpr int qq = decltype(qc)::value;
      if (kt + qq < nst) pp.template stage_s<qq % P::U>(kt + qq, nst, false);
    });
  }
  if (half_tail) {  // K % 64 == 32: one 32-wide sub-stage into slot 0, unpipelined
    const char* xb = pp.xbase + (size_t)nst * (kBK * 2);
    const char* wb = pp.wbase + (size_t)nst * (kBK * 2);
#pragma unroll
    for (int d = 0; d < P::DPW; ++d) {
      const int D = wave + 8 * d, G = d < XPW ? D : D - XG;
      const uint32_t chunk = (uint32_t)((lane & 7) ^ (((8 * G + (lane >> 3)) >> 1) & 7));
      if (chunk < 4) {
        if (d < XPW)
          dma16(pp.lds_addr + pp.dlds[d], pp.doff[d], xb);
        else
          dma16(pp.lds_addr + P::WRING + pp.dlds[d], pp.doff[d], wb);
      }
    }
    wait_vm<0>();
    __syncthreads();
    const uint32_t b0 = pp.lds_addr + pp.xrow + pp.a0;
    const uint32_t w0 = pp.lds_addr + P::WRING + pp.wrow + pp.a0;
    h8 wf[FN];
    static_for<0, FN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      ds_read16<j * 16 * 128>(wf[j], w0);
    });
    static_for<0, FM>([&](auto fc) {
      constexpr int i = decltype(fc)::value;
      h8 a;
      ds_read16<i * 16 * 128>(a, b0);
      wait_lgkm<0>();
      tie(a);
      if constexpr (i == 0) {
#pragma unroll
        for (int j = 0; j < FN; ++j) tie(wf[j]);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) mfma_acc_v(pp.acc[i][j], a, wf[j]);
    });
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  store_tile8<FM, FN, BN, FNA % 2 == 0 && FNB % 2 == 0>(pp.acc, p, mi, split, m0, n0, rbase, cbase, r, g, (float*)lds);
}

template <int FM, int FNA, int FNB>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void gemm_tile8_kernel(const TileArgs p) {
  constexpr int BN = 32 * (FNA + FNB), BM = 32 * FM;
  constexpr int LDSB = 2 * BM * 128 + 3 * BN * 128;
  static_assert(LDSB <= 160 * 1024, "the rings fit the LDS");
  static_assert(LDSB >= 128 * (BN + 4) * 4, "the epilogue's staging fits the rings");
  static_assert(LDSB >= BM * (BN / 2 + 8) * 2, "the fp16 SwiGLU staging fits the rings");
  __shared__ __attribute__((aligned(1024))) char lds[LDSB];
  uint32_t mt, gs, split;
  tile_coords(p, xcd_remap(blockIdx.x, gridDim.x), mt, gs, split);
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxMembers; ++i)
    if (i < (int)p.count && gs >= p.mem[i].stripe_begin) mi = i;
  const uint32_t ldw = p.mem[mi].ldw, N = p.mem[mi].n;
  const uint32_t m0 = mt * BM, n0 = (gs - p.mem[mi].stripe_begin) * BN;
  const uint32_t kb = split * p.kps;
  const uint32_t ke = min(p.k, kb + p.kps);
  const int nst = (int)((ke - kb) / kBK);
  const bool half_tail = ((ke - kb) % kBK) != 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave < 4)
    tile8_wave<FM, FNA, FNA, FNB, 0>(p, lds, wave, mi, m0, n0, split, nst, half_tail, ldw, N, kb);
  else
    tile8_wave<FM, FNB, FNA, FNB, 4>(p, lds, wave, mi, m0, n0, split, nst, half_tail, ldw, N, kb);
}

// ---- the compiled menu: (FM, NBX, NBW). BM = 16·FM rows, BN = 256.
#define DH_TILE_MENU(X) \
  X(1, 3, 3)            \
  X(2, 3, 3)            \
  X(4, 3, 3)            \
  X(6, 3, 3)            \
  X(8, 3, 3)            \
  X(10, 3, 3)           \
  X(13, 2, 3)           \
  X(5, 3, 3)            \
  X(7, 3, 3)            \
  X(11, 2, 3)

struct VariantEntry {
  VariantInfo info;
  void (*fn)(const TileArgs);
};

#define DH_TILE_ENTRY(FM, NBX, NBW) {{FM, 4, 4, 1}, gemm_tile_kernel<FM, NBX, NBW>},
static const VariantEntry kVariants[] = {
    DH_TILE_MENU(DH_TILE_ENTRY)
    // 96 x 160 with a 5-deep ring: small M (48-96 rows) over wide N; swapped operands, epilogue from registers
    {{3, 5, 2, 2}, gemm_tile22_kernel<3, 5, 5, 5, true>},
    // 160 x 288: at M ≈ 603 the gate|up projection is 4 x 64 = 256 tiles, one per CU
    {{5, 9, 2, 2}, gemm_tile22_kernel<5, 9, 2, 3>},
    // 288 x 224 and 224 x 224: the M = 2307 projections in fewer rounds of 256 tiles
    {{9, 7, 2, 2}, gemm_tile22_kernel<9, 7, 2, 3>},
    {{7, 7, 2, 2}, gemm_tile22_kernel<7, 7, 2, 3>},
    // 160 x 160: the N = 2560 projections (10 % less LDS traffic per output than 96 x 256); swapped operands,
    // epilogue from registers
    {{5, 5, 2, 2}, gemm_tile22_kernel<5, 5, 3, 3, true>},
    // 128 x 96 with a 5-deep ring: medium M (96-490 rows) over narrow N
    {{4, 3, 2, 2}, gemm_tile22_kernel<4, 3, 5, 5>},
    // 8 waves, two per SIMD: 256 x 256 and 256 x 224, the wide M = 2307 projections in under three rounds
    {{8, 8, 2, 2, 2}, gemm_tile8_kernel<8, 4, 4>},
    {{8, 7, 2, 2, 2}, gemm_tile8_kernel<8, 4, 3>},
};
#undef DH_TILE_ENTRY

static_assert(sizeof(kVariants) / sizeof(kVariants[0]) <= 24, "kernel ids from 24 on name the other kernels");
int variant_count() { return (int)(sizeof(kVariants) / sizeof(kVariants[0])); }
VariantInfo variant_info(int v) { return kVariants[v].info; }

hipError_t launch_tile(int v, const TileArgs& a, uint32_t grid, hipStream_t s) {
  const VariantEntry& e = kVariants[v];
  hipLaunchKernelGGL(e.fn, dim3(grid), dim3(64 * e.info.waves()), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Split-K reduction: y = epi(Σ_s ws[s]) summed in split order (deterministic).
// One thread per 4 consecutive outputs: 16-byte partial reads.
__global__ void splitk_reduce_kernel(const float* __restrict__ ws, uint32_t splits, uint32_t m, uint32_t n, void* y,
                                     uint32_t ldy, uint32_t epi) {
  const uint32_t ncols = epi == 3u ? n / 2 : n;
  const size_t total = (size_t)m * (ncols / 4);
  const size_t plane = (size_t)m * n;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(t / (ncols / 4)), oc = (uint32_t)(t % (ncols / 4)) * 4;
    f4 v;
    if (epi == 3u) {
      const uint32_t gc = (oc / kSwigluBlock) * 2 * kSwigluBlock + oc % kSwigluBlock;
      const float* pg = ws + (size_t)row * n + gc;
      f4 gs = *(const f4*)pg, us = *(const f4*)(pg + kSwigluBlock);
      for (uint32_t s = 1; s < splits; ++s) {
        gs += *(const f4*)(pg + s * plane);
        us += *(const f4*)(pg + s * plane + kSwigluBlock);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = swiglu_f(gs[q], us[q]);
    } else {
      const float* pp = ws + (size_t)row * n + oc;
      v = *(const f4*)pp;
      for (uint32_t s = 1; s < splits; ++s) v += *(const f4*)(pp + s * plane);
    }
    const size_t o = (size_t)row * ldy + oc;
    typedef float fl2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    if (epi == 0u || epi == 2u) {
      float* dst = (float*)y + o;  // 8-byte aligned (contract): two float2 accesses
      fl2 lo = fl2{v[0], v[1]}, hi = fl2{v[2], v[3]};
      if (epi == 2u) {
        lo += *(const fl2*)dst;
        hi += *(const fl2*)(dst + 2);
      }
      *(fl2*)dst = lo;
      *(fl2*)(dst + 2) = hi;
    } else {
      _Float16* dst = (_Float16*)y + o;  // 4-byte aligned (contract)
      *(h2*)dst = h2{(_Float16)v[0], (_Float16)v[1]};
      *(h2*)(dst + 2) = h2{(_Float16)v[2], (_Float16)v[3]};
    }
  }
}

hipError_t launch_splitk_reduce(const float* ws, uint32_t splits, uint32_t m, uint32_t n, void* y, uint32_t ldy,
                                uint32_t epi, hipStream_t s) {
  const size_t total = (size_t)m * ((epi == 3u ? n / 2 : n) / 4);
  const uint32_t blocks = (uint32_t)std::min<size_t>((total + 255) / 256, 16384);
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
    ((_Float16*)y)[o] = (_Float16)swiglu_f(dot(gc), dot(gc + kSwigluBlock));
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
  if (ncols == 0) return hipSuccess;
  hipLaunchKernelGGL(gemm_reference_kernel, dim3((ncols + 127) / 128, std::min<uint32_t>(m, 4096)), dim3(128), 0, s, x, ldx, w, ldw, y, ldy, m,
                     n, k, epi);
  return hipGetLastError();
}

}  // namespace dh
