// GEMM launch planner for MI355X: (m, n, k, epi) → tile variant + split-K.
// decide's counterpart is gemm_configs::plan / recommend
// (crates/decide-metal/src/gemm_configs.rs:290-314), a table measured on an
// M1 Pro. This one is a table measured on an MI355X for decide's engine
// shapes, with a calibrated cost model (rounds of 256 workgroups, per-stage
// time per tile height, HBM floor, split-K reduction) for every other shape.
// Pure host code: no device needed.
#pragma once

#include <stdint.h>

namespace dh {

struct Plan {
  int variant;
  uint32_t splits;
  uint32_t kps;       // K per split (multiple of 64)
  uint32_t mtiles, stripes;
  uint32_t grid;      // workgroups of the tile kernel
  uint64_t ws_bytes;  // split-K workspace
  double est_us;      // model estimate
};

// Plan.variant of the small-M weight-streaming kernel (gemm_stream.hip): 32
// output columns per workgroup, M <= 16, K a multiple of 128.
constexpr int kStreamVariant = 64;  // DH_GEMM_STREAM_VARIANT
constexpr uint32_t kStreamMaxM = 16;
// Widest N (summed over a grouped launch's members) the streaming kernel takes:
// measured faster than the FM = 1/2 tile variants with split-K up to here
// (k|v, o and down of the pruned layer) and slower beyond (q|gate, gate|up).
constexpr uint32_t kStreamMaxN = 4096;

// Model estimate for one (variant, splits) choice; +inf if the choice is not
// valid for the shape.
double plan_estimate_us(int variant, uint32_t splits, uint32_t m, uint32_t n, uint32_t k, uint32_t epi);
// Builds the plan for (variant, splits), filling the derived fields.
Plan plan_make(int variant, uint32_t splits, uint32_t m, uint32_t n, uint32_t k, uint32_t epi);
// The weight-streaming kernel's plan (M <= kStreamMaxM, K % 128 == 0, N % 32 == 0).
Plan plan_stream(uint32_t m, uint32_t n, uint32_t k, uint64_t max_ws);
// Best plan for a single GEMM. `max_ws` caps the split-K workspace bytes.
Plan plan_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t epi, uint64_t max_ws);
// The largest split-K workspace plan_gemm asks for over every M in 1..max_m and
// every epilogue at (n, k): the workspace a caller must hold so that no call of
// up to max_m rows grows it. The table switches split counts between measured
// rows, so the need is not monotone in M; this sweeps every M.
uint64_t plan_ws_need(uint32_t max_m, uint32_t n, uint32_t k, uint64_t max_ws);
// Best plan for a grouped launch of `count` members of widths ns[] that share
// X (no split-K). Each member rounds up to whole column stripes of its own.
Plan plan_grouped(uint32_t m, uint32_t k, const uint32_t* ns, uint32_t count);
// The tile kernels' work order for plan p (TileArgs::ngroup): the hardware
// deals workgroups to the 8 XCDs round-robin and xcd_remap gives each XCD a
// contiguous run of work ids, so the order decides which X row blocks and W
// column stripes share one XCD's L2. Returns the stripe-group width (0 = M
// tiles fastest) that minimises the bytes of distinct X and W tiles each XCD
// fetches per round of one workgroup per CU, over a few candidates.
// DH_GEMM_TILE_GROUP=<g> (0..64) in the environment fixes it (for measurements).
uint32_t plan_order(const Plan& p);

}  // namespace dh
