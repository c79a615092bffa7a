// Launch-argument structs and launcher declarations shared by the HIP kernel
// sources and the C-ABI layer (api.cpp). Host-visible, no device code here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dh {

constexpr int kMaxMembers = 8;
constexpr int kBK = 64;  // K extent of one pipeline stage of the tile kernel
constexpr uint32_t kSwigluBlock = 16;  // gate|up interleave block (decide's SWIGLU_BLOCK)

// The file-scope device scratch of the no-allocation GEMM entry point
// (noalloc.hip): split-K partials up to this many bytes.
constexpr uint64_t kNoAllocScratchBytes = 48ull << 20;
// Its device address on `device` (which must be current), looked up once per device.
hipError_t noalloc_scratch(int device, float** out);

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
  uint32_t ngroup;    // work order within a split: 0 = M tiles fastest; g > 0 = the stripes in groups of g, and
                      // within a group the stripes fastest, then the M tiles (see tile_coords in gemm_tile.hip)
  uint32_t count;     // members in use
  Member mem[kMaxMembers];
};

// Geometry of one compiled tile variant.
struct VariantInfo {
  int fm;  // 16-row fragments per wave
  int fn;  // 16-column fragments per wave
  int wn;  // waves along N
  int wm;  // waves along M
  int spw = 1;  // waves per wave position (2: each position's block split between two waves of one SIMD)
  int bm() const { return 16 * fm * wm; }
  int bn() const { return 16 * fn * wn; }
  int waves() const { return wm * wn * spw; }
};

// The small-M weight-streaming kernel (gemm_stream.hip) over the members of
// `a`: a.nstripes counts 32-column blocks (mem[i].stripe_begin in those
// units), a.kps is a multiple of 128, grid = a.nstripes · a.splits.
hipError_t launch_stream(const TileArgs& a, uint32_t grid, hipStream_t s);

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
// x[r] += Σ_s ws[s][r] (split-K partials [splits][rows][h], split order), then y[r] = rmsnorm(x[r]): bitwise the
// split-K reduce's AddF32 followed by launch_rmsnorm_rows, for the shapes splitk_add_rmsnorm_fits accepts.
bool splitk_add_rmsnorm_fits(uint32_t splits, uint32_t h, uint32_t ldx, uint32_t ldy, const void* x, const void* w,
                             const void* y);
hipError_t launch_splitk_add_rmsnorm(const float* ws, uint32_t splits, uint32_t rows, uint32_t h, float* x,
                                     uint32_t ldx, const float* w, _Float16* y, uint32_t ldy, bool add_one, float eps,
                                     hipStream_t s);
hipError_t launch_fill_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, float std, hipStream_t s);
hipError_t launch_fill_normal(void* out, uint64_t n, uint64_t seed, float mean, float sd, uint32_t dtype,
                              hipStream_t s);

// ---- the non-GEMM forward kernels (mixer.hip, attention.hip)
hipError_t launch_conv_silu_l2(const float* p, const float* prev, const float* w, float* q, float* k, float* v,
                               uint32_t t, uint32_t ldp, hipStream_t s);
hipError_t launch_conv_state_update(const float* p, const float* prev_in, float* prev_out, uint32_t t, uint32_t ldp,
                                    hipStream_t s);
hipError_t launch_gated_delta(const float* q, const float* k, const float* v, const float* a, const float* b,
                              const float* a_log, const float* dt_bias, const float* state_in, float* state_out,
                              float* o, uint32_t t, uint32_t ldab, bool write_state, hipStream_t s);
// The chunked recurrence (delta_chunk.hip): `ws` holds delta_chunk_ws_floats(t) floats.
size_t delta_chunk_ws_floats(uint32_t t);
hipError_t launch_gated_delta_chunked(const float* q, const float* k, const float* v, const float* a, const float* b,
                                      const float* a_log, const float* dt_bias, const float* state_in,
                                      float* state_out, float* o, float* ws, uint32_t t, uint32_t ldab,
                                      bool write_state, hipStream_t s);
// The conv step fused into the chunked recurrence: from the raw in-projection
// p (row stride ldp), the conv state `prev` [3][8192] and the conv weights;
// q (the conv step's q output) is written for the scan, k and v are not.
hipError_t launch_conv_gated_delta_chunked(const float* p, const float* prev, const float* conv_w, uint32_t ldp,
                                           float* q, const float* a, const float* b, uint32_t ldab,
                                           const float* a_log, const float* dt_bias, const float* state_in,
                                           float* state_out, float* o, float* ws, uint32_t t, bool write_state,
                                           hipStream_t s);
hipError_t launch_gated_rmsnorm_silu(const float* o, const float* z, const float* w, _Float16* y, uint32_t t,
                                     uint32_t ldz, hipStream_t s);
hipError_t launch_q_norm_rope(const float* pq, const float* qw, const float* inv_freq, const uint32_t* qpos,
                              _Float16* qo, uint32_t rows, uint32_t ldq, hipStream_t s);
hipError_t launch_kv_norm_rope(const float* pkv, const float* kw, const float* inv_freq, _Float16* kc, _Float16* vc,
                               uint32_t rows, uint32_t ldkv, uint32_t kcol, uint32_t vcol, uint32_t pos0,
                               hipStream_t s);
// Attention's key pieces: each query block's keys are cut every L blocks of 32
// keys into at most np pieces (np = 1: no cut, no workspace).
struct AttnSplit {
  uint32_t L = 2;
  uint32_t np = 1;
};
constexpr uint32_t kAttnMaxPieces = 16;       // pieces per query block
constexpr uint32_t kAttnMaxPieceRows = 5120;  // query-block rows x pieces with partial state (the workspace bound)
// The cut for `rows` query rows whose positions are below npos, on `cus` CUs.
AttnSplit attention_split(uint32_t rows, uint32_t npos, uint32_t cus);
// Workspace bytes the cut needs (the pieces' partial states), 0 for np = 1.
uint64_t attention_ws_bytes(uint32_t rows, const AttnSplit& sp);
// The most any cut for up to max_rows query rows can need (at most 84.5 MB).
uint64_t attention_ws_max(uint32_t max_rows);
hipError_t launch_attention(const _Float16* q, const _Float16* kc, const _Float16* vc, const float* pq,
                            const uint32_t* qpos, _Float16* y, float* part, uint32_t rows, uint32_t ldq,
                            const AttnSplit& sp, hipStream_t s);
hipError_t launch_embed_bf16(const uint32_t* ids, const uint16_t* table, float* out, uint32_t t, uint32_t h,
                             hipStream_t s);

}  // namespace dh
