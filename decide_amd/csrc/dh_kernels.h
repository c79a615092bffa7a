// Launch-argument structs and launcher declarations shared by the HIP kernel
// sources and the C-ABI layer (api.cpp). Host-visible, no device code here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dh {

constexpr int kMaxMembers = 8;
constexpr int kBK = 64;  // K extent of one pipeline stage of the tile kernel
constexpr uint32_t kSwigluBlock = 16;  // gate|up interleave block (decide's SWIGLU_BLOCK)

// One output of a (grouped) tile launch: Y = epi(X · Wᵀ) for one weight.
struct Member {
  const _Float16* w;  // [n, k], row stride ldw
  void* y;            // output, row stride ldy (elements of the output type)
  uint32_t ldw, ldy, n, epi;
  uint32_t stripe_begin;  // first global column stripe of this member
  uint32_t pad_;
};

// Everything one launch of the tile kernel needs (passed by value as the
// kernel argument; 8 members keep it well under the kernarg limit).
struct TileArgs {
  const _Float16* x;  // [m, k], row stride ldx, shared by every member
  float* ws;          // split-K partials [splits][m][n] fp32 (single member), or null
  uint32_t ldx, m, k;
  uint32_t mtiles;    // ceil(m / BM)
  uint32_t splits;    // split-K factor
  uint32_t kps;       // K per split (a multiple of kBK)
  uint32_t nstripes;  // column stripes summed over the members
  uint32_t count;     // members in use
  Member mem[kMaxMembers];
};

// Geometry of one compiled tile variant.
struct VariantInfo {
  int fm;  // 16-row fragments per wave (and per workgroup: waves split N only)
  int fn;  // 16-column fragments per wave
  int wn;  // waves per workgroup
  int bm() const { return 16 * fm; }
  int bn() const { return 16 * fn * wn; }
};

int variant_count();
VariantInfo variant_info(int v);
// Enqueues the tile kernel of variant v over `grid` workgroups.
hipError_t launch_tile(int v, const TileArgs& a, uint32_t grid, hipStream_t s);

// Sums split-K partials in split order and applies the epilogue.
hipError_t launch_splitk_reduce(const float* ws, uint32_t splits, uint32_t m, uint32_t n, void* y, uint32_t ldy,
                                uint32_t epi, hipStream_t s);

// The simple M-independent kernel (one output per thread, K in order).
hipError_t launch_gemm_reference(const _Float16* x, uint32_t ldx, const _Float16* w, uint32_t ldw, void* y,
                                 uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi, hipStream_t s);

hipError_t launch_gather_rows(const void* x, const uint32_t* rowmap, void* out, uint32_t rows, uint32_t h,
                              uint32_t elem_bytes, hipStream_t s);
hipError_t launch_final_head(const float* x, const float* w, const uint16_t* table, const uint32_t* cand,
                             const uint32_t* ncand, float* logits, uint32_t rows, uint32_t hidden,
                             uint32_t max_cand, float eps, hipStream_t s);
hipError_t launch_rmsnorm_rows(const float* x, const float* w, _Float16* y, const uint32_t* rowmap, uint32_t rows,
                               uint32_t h, uint32_t ld_in, uint32_t ld_out, bool add_one, float eps, hipStream_t s);
hipError_t launch_fill_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, float std, hipStream_t s);

}  // namespace dh
