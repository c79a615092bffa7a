// See plan.h. Two parts:
//   * a table measured on an MI355X (decide_amd/tune_gemm.py): for decide's
//     engine shapes (K, N) at M in {1, 3, 8, 16, 24, 48, 96, 163, 276, 490,
//     603, 1024, 2307}, the fastest (tile variant, split-K) with weights
//     streaming from HBM — the MI355X counterpart of decide's M1 Pro
//     RECOMMENDED table (crates/decide-metal/src/gemm_configs.rs:247-283);
//   * a cost model for every other shape, calibrated on the same
//     measurements: a 64-wide K stage of a BM = 16·FM tile takes about
//     0.115·FM µs (MFMA issue plus the DMA and barrier it waits on), blocks
//     run in rounds of 256 (one per CU), the weights stream at most at
//     6 TB/s, and split-K adds a reduction pass over S + 2 fp32 planes.
// The table entry is used when the requested M is within 12 % of a measured
// M for that (K, N); otherwise the model picks the variant and split. Apart
// from both, plan_order picks the tiles' work order for the XCDs' L2s.
#include "plan.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <limits>

#include "dh_kernels.h"

namespace dh {

namespace {
constexpr double kCUs = 256.0;
constexpr double kHbmBps = 6.0e12;      // sustained HBM read bandwidth (measured streaming copy)
constexpr double kStageUsPerFM = 0.115;  // µs per 64-wide stage per 16-row fragment
constexpr double kMinStageUs = 0.35;     // a stage is never cheaper than its DMA round trip
constexpr double kLaunchUs = 3.0;        // kernel launch + prologue + epilogue
constexpr uint32_t kSplitMenu[] = {1, 2, 3, 4, 6, 8};

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

struct Measured {
  uint32_t k, n, m;
  int variant;
  uint32_t splits;
};

// {k, n, m, variant, splits}: fastest on an MI355X (gfx950, 256 CUs), the
// variant index into the compiled menu (gemm_tile.hip: 4 waves in a row with
// FM 1, 2, 4, 6, 8, 10, 13, 5, 7, 11; then 2 x 2 tiles 96 x 160 (5-deep ring),
// 160 x 288, 288 x 224, 224 x 224, 160 x 160 and 128 x 96 (5-deep ring)),
// weights rotated over > 256 MB. Regenerate with `python -m
// decide_amd.tune_gemm` after any change to the tile kernel. Three rows are
// checked against sustained runs instead, because the chip is power-limited
// there and burst timings can rank close choices differently: the C2 down row
// in the bench's gate|up + down loop, and the M = 2307 gate|up and q|gate|k|v
// rows in the 36-layer forward, where the burst-fastest 160 x 288 / 224 x 224
// tiles (within 1-2 % of these in the tuner) made the forward 0.3 ms slower.
const Measured kMeasured[] = {
    {2560, 12352, 1, 0, 4},  // 16.86 us
    {2560, 12352, 3, 0, 4},  // 17.02 us
    {2560, 12352, 8, 0, 4},  // 17.08 us
    {2560, 12352, 16, 0, 4},  // 17.71 us
    {2560, 12352, 24, 1, 4},  // 18.56 us
    {2560, 12352, 48, 7, 4},  // 21.04 us
    {2560, 12352, 96, 10, 3},  // 24.07 us
    {2560, 12352, 163, 3, 2},  // 32.2 us
    {2560, 12352, 276, 10, 1},  // 35.54 us
    {2560, 12352, 490, 8, 1},  // 44.43 us
    {2560, 12352, 603, 4, 1},  // 48.46 us
    {2560, 12352, 1024, 17, 1},  // 67.2 us (8-wave 256 x 224; 72.1 for 208 x 256 beside it)
    {2560, 12352, 2307, 16, 1},  // 146.9 us (8-wave 256 x 256; 159.6 for the 160 x 256 tile beside it)
    {2560, 10240, 1, 0, 4},  // 15.56 us
    {2560, 10240, 3, 0, 4},  // 15.69 us
    {2560, 10240, 8, 0, 4},  // 16.18 us
    {2560, 10240, 16, 0, 4},  // 16.64 us
    {2560, 10240, 24, 1, 4},  // 17.19 us
    {2560, 10240, 48, 10, 4},  // 18.62 us
    {2560, 10240, 96, 10, 4},  // 21.75 us
    {2560, 10240, 163, 15, 1},  // 24.66 us
    {2560, 10240, 276, 3, 2},  // 33.22 us
    {2560, 10240, 490, 14, 1},  // 37.89 us
    {2560, 10240, 603, 14, 1},  // 41.27 us
    {2560, 10240, 1024, 9, 1},  // 58.28 us
    {2560, 10240, 2307, 17, 1},  // 126.0 us (8-wave 256 x 224; 134.5 for 208 x 256 beside it)
    {2560, 18432, 1, 0, 3},  // 22.01 us
    {2560, 18432, 3, 0, 3},  // 22.27 us
    {2560, 18432, 8, 0, 3},  // 22.66 us
    {2560, 18432, 16, 0, 3},  // 23.24 us
    {2560, 18432, 24, 1, 3},  // 23.98 us
    {2560, 18432, 48, 10, 2},  // 25.43 us
    {2560, 18432, 96, 10, 2},  // 29.49 us
    {2560, 18432, 163, 10, 1},  // 34.79 us
    {2560, 18432, 276, 14, 1},  // 38.59 us
    {2560, 18432, 490, 9, 1},  // 50.79 us
    {2560, 18432, 603, 11, 1},  // 56.4 us
    {2560, 18432, 1024, 5, 1},  // 90.81 us
    {2560, 18432, 2307, 16, 1},  // 194.2 us (8-wave 256 x 256; 209.6 for 176 x 256 beside it)
    {4096, 2560, 1, 0, 8},  // 12.91 us
    {4096, 2560, 3, 0, 8},  // 13.32 us
    {4096, 2560, 8, 0, 8},  // 13.54 us
    {4096, 2560, 16, 0, 8},  // 14.09 us
    {4096, 2560, 24, 0, 8},  // 14.1 us
    {4096, 2560, 48, 0, 8},  // 14.41 us
    {4096, 2560, 96, 1, 6},  // 16.02 us
    {4096, 2560, 163, 15, 4},  // 16.97 us
    {4096, 2560, 276, 15, 3},  // 18.96 us
    {4096, 2560, 490, 15, 2},  // 24.42 us
    {4096, 2560, 603, 14, 4},  // 26.99 us
    {4096, 2560, 1024, 14, 2},  // 37.08 us (39.33 for 96 x 256, split 2, beside it)
    {4096, 2560, 2307, 14, 1},  // 58.62 us (60.67 for 96 x 256 beside it; same bits)
    {9216, 2560, 1, 0, 8},  // 20.67 us
    {9216, 2560, 3, 0, 8},  // 20.83 us
    {9216, 2560, 8, 0, 8},  // 21.44 us
    {9216, 2560, 16, 0, 8},  // 22.18 us
    {9216, 2560, 24, 0, 8},  // 21.73 us
    {9216, 2560, 48, 0, 8},  // 21.94 us
    {9216, 2560, 96, 15, 8},  // 21.03 us
    {9216, 2560, 163, 10, 8},  // 24.88 us
    {9216, 2560, 276, 15, 3},  // 28.89 us
    {9216, 2560, 490, 4, 6},  // 38.05 us
    {9216, 2560, 603, 14, 4},  // 40.87 us; also the best in the bench's sustained gate|up + down loop
    {9216, 2560, 1024, 4, 3},  // 59.23 us
    {9216, 2560, 2307, 14, 1},  // 110.49 us
    {2560, 2048, 1, 0, 8},  // 11.62 us
    {2560, 2048, 3, 0, 8},  // 11.76 us
    {2560, 2048, 8, 0, 8},  // 12.25 us
    {2560, 2048, 16, 0, 8},  // 12.51 us
    {2560, 2048, 24, 0, 8},  // 12.52 us
    {2560, 2048, 48, 0, 8},  // 12.95 us
    {2560, 2048, 96, 0, 4},  // 13.69 us
    {2560, 2048, 163, 15, 4},  // 14.26 us
    {2560, 2048, 276, 15, 3},  // 15.56 us
    {2560, 2048, 490, 15, 2},  // 19.73 us
    {2560, 2048, 603, 15, 2},  // 20.02 us
    {2560, 2048, 1024, 2, 2},  // 26.91 us
    {2560, 2048, 2307, 14, 1},  // 38.24 us
    {2560, 8192, 1, 0, 6},  // 14.61 us
    {2560, 8192, 3, 0, 6},  // 14.82 us
    {2560, 8192, 8, 0, 6},  // 15.11 us
    {2560, 8192, 16, 0, 6},  // 15.2 us
    {2560, 8192, 24, 0, 4},  // 15.61 us
    {2560, 8192, 48, 1, 4},  // 16.91 us
    {2560, 8192, 96, 2, 4},  // 19.48 us
    {2560, 8192, 163, 3, 4},  // 23.91 us
    {2560, 8192, 276, 7, 2},  // 29.67 us
    {2560, 8192, 490, 14, 1},  // 36.36 us
    {2560, 8192, 603, 7, 1},  // 40.7 us
    {2560, 8192, 1024, 4, 1},  // 48.01 us
    {2560, 8192, 2307, 5, 1},  // 104.68 us
    {2560, 6144, 1, 0, 6},  // 13.37 us
    {2560, 6144, 3, 0, 6},  // 13.61 us
    {2560, 6144, 8, 0, 6},  // 14.19 us
    {2560, 6144, 16, 0, 8},  // 14.3 us
    {2560, 6144, 24, 0, 4},  // 15.02 us
    {2560, 6144, 48, 1, 4},  // 16.12 us
    {2560, 6144, 96, 15, 4},  // 16.92 us
    {2560, 6144, 163, 15, 2},  // 19.03 us
    {2560, 6144, 276, 15, 1},  // 22.95 us
    {2560, 6144, 490, 15, 1},  // 28.5 us
    {2560, 6144, 603, 2, 1},  // 36.14 us
    {2560, 6144, 1024, 8, 1},  // 42.53 us
    {2560, 6144, 2307, 12, 1},  // 81.32 us
    {2560, 9216, 1, 0, 6},  // 14.91 us
    {2560, 9216, 3, 0, 6},  // 15.06 us
    {2560, 9216, 8, 0, 4},  // 15.55 us
    {2560, 9216, 16, 0, 6},  // 15.89 us
    {2560, 9216, 24, 1, 6},  // 16.62 us
    {2560, 9216, 48, 10, 4},  // 17.9 us
    {2560, 9216, 96, 10, 4},  // 20.86 us
    {2560, 9216, 163, 15, 1},  // 24.05 us
    {2560, 9216, 276, 14, 2},  // 30.94 us
    {2560, 9216, 490, 14, 1},  // 36.95 us
    {2560, 9216, 603, 14, 1},  // 41.11 us
    {2560, 9216, 1024, 5, 1},  // 53.1 us
    {2560, 9216, 2307, 9, 1},  // 114.62 us
};
}  // namespace

Plan plan_make(int variant, uint32_t splits, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  const VariantInfo v = variant_info(variant);
  Plan p{};
  p.variant = variant;
  const uint32_t stages = ceil_div(k, kBK);
  splits = std::max(1u, std::min(splits, std::max(stages, 1u)));
  p.kps = ceil_div(stages, splits) * kBK;
  p.splits = p.kps ? ceil_div(k, p.kps) : 1;  // splits that would be empty are dropped; K = 0: one, empty
  p.mtiles = ceil_div(m, (uint32_t)v.bm());
  p.stripes = ceil_div(n, (uint32_t)v.bn());
  p.grid = p.mtiles * p.stripes * p.splits;
  p.ws_bytes = p.splits > 1 ? (uint64_t)p.splits * m * n * sizeof(float) : 0;
  p.est_us = plan_estimate_us(variant, p.splits, m, n, k, epi);
  return p;
}

double plan_estimate_us(int variant, uint32_t splits, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  const VariantInfo v = variant_info(variant);
  const uint32_t stages = ceil_div(k, kBK);
  if (splits < 1 || splits > stages) return std::numeric_limits<double>::infinity();
  const uint32_t st_per_split = ceil_div(stages, splits);
  splits = ceil_div(stages, st_per_split);
  const double mtiles = ceil_div(m, (uint32_t)v.bm()), stripes = ceil_div(n, (uint32_t)v.bn());
  const double blocks = mtiles * stripes * splits;
  const double rounds = std::ceil(blocks / kCUs);
  // MFMAs per wave per stage, in units of a 16-row fragment of the 4-fragment-wide waves
  const double stage_us = std::max(kMinStageUs, kStageUsPerFM * v.fm * v.fn / 4.0);
  const double compute_us = rounds * st_per_split * stage_us;
  const double out_b = (epi == 0u || epi == 2u) ? 4.0 : 2.0;
  const double out_cols = epi == 3u ? n / 2.0 : n;
  const double hbm_us = (2.0 * n * k + 2.0 * m * k + out_b * m * out_cols) / kHbmBps * 1e6;
  double t = std::max(compute_us, hbm_us) + kLaunchUs;
  if (splits > 1) t += kLaunchUs + (splits + 2.0) * m * n * 4.0 / kHbmBps * 1e6;
  return t;
}

namespace {
Plan plan_model(uint32_t m, uint32_t n, uint32_t k, uint32_t epi, uint64_t max_ws) {
  Plan best{};
  best.est_us = std::numeric_limits<double>::infinity();
  best.variant = -1;
  for (int v = 0; v < variant_count(); ++v) {
    for (uint32_t s : kSplitMenu) {
      const double t = plan_estimate_us(v, s, m, n, k, epi);
      if (!(t < best.est_us)) continue;
      const Plan p = plan_make(v, s, m, n, k, epi);
      if (p.ws_bytes > max_ws) continue;
      best = p;
    }
  }
  return best;
}
}  // namespace

// The weight-streaming kernel for M <= 16: one workgroup per 32 columns and
// K split, splits chosen so that about two workgroups per CU stream at once
// (each split a whole number of 128-wide k blocks; no split when the
// workspace is capped, as for grouped launches).
Plan plan_stream(uint32_t m, uint32_t n, uint32_t k, uint64_t max_ws) {
  Plan p{};
  p.variant = kStreamVariant;
  const uint32_t blocks = n / 32, kb = k / 128;
  uint32_t s = std::min(std::max(1u, ceil_div(512, blocks)), kb);
  const uint32_t kpb = ceil_div(kb, s);
  s = ceil_div(kb, kpb);
  p.splits = s;
  p.kps = kpb * 128;
  p.ws_bytes = s > 1 ? (uint64_t)s * m * n * 4 : 0;
  if (p.ws_bytes > max_ws) {
    p.splits = 1;
    p.kps = k;
    p.ws_bytes = 0;
  }
  p.mtiles = 1;
  p.stripes = blocks;
  p.grid = blocks * p.splits;
  p.est_us = (double)n * k * 2 / kHbmBps * 1e6 + kLaunchUs;
  return p;
}

Plan plan_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t epi, uint64_t max_ws) {
  // decide's contract admits N = 0 (nothing to launch: an empty grid) and K = 0 (the tiles run no
  // stage and store the empty sum).
  if (n == 0 || k == 0) return plan_make(0, 1, m, n, k, epi);
  if (m <= kStreamMaxM && n <= kStreamMaxN && k % 128 == 0 && n % 32 == 0) return plan_stream(m, n, k, max_ws);
  const Measured* near = nullptr;
  double best_rel = 0.12;
  for (const Measured& e : kMeasured) {
    if (e.k != k || e.n != n || e.variant >= variant_count()) continue;
    const double rel = std::fabs((double)m - e.m) / e.m;
    if (rel <= best_rel) {
      best_rel = rel;
      near = &e;
    }
  }
  if (near) {
    const Plan p = plan_make(near->variant, near->splits, m, n, k, epi);
    if (p.ws_bytes <= max_ws) return p;
  }
  return plan_model(m, n, k, epi, max_ws);
}

uint64_t plan_ws_need(uint32_t max_m, uint32_t n, uint32_t k, uint64_t max_ws) {
  uint64_t need = 0;
  for (uint32_t m = 1; m <= max_m; ++m)
    for (uint32_t epi = 0; epi < 4; ++epi) need = std::max(need, plan_gemm(m, n, k, epi, max_ws).ws_bytes);
  return need;
}

Plan plan_grouped(uint32_t m, uint32_t k, const uint32_t* ns, uint32_t count) {
  // Members share X and launch together: plan as one GEMM of the summed width
  // (the table's row for that width is measured on the grouped launch where
  // the engine has one), unless the members' own stripe rounding would add a
  // round of 256 tiles to that plan; then the model picks, counting the
  // stripes member by member.
  uint32_t n_total = 0;
  for (uint32_t i = 0; i < count; ++i) n_total += ns[i];
  const Plan p = plan_gemm(m, n_total, k, 0u, 0);
  if (p.variant == kStreamVariant) return p;
  // the width whose single-GEMM stripe count equals the grouped one for variant v
  auto grouped_n = [&](int v) {
    const uint32_t bn = (uint32_t)variant_info(v).bn();
    uint32_t s = 0;
    for (uint32_t i = 0; i < count; ++i) s += ceil_div(ns[i], bn);
    return s * bn;
  };
  const uint32_t cus = (uint32_t)kCUs;
  const uint32_t bn = (uint32_t)variant_info(p.variant).bn();
  if (ceil_div(p.mtiles * (grouped_n(p.variant) / bn), cus) <= ceil_div(p.grid, cus)) return p;
  Plan best = p;
  double best_us = std::numeric_limits<double>::infinity();
  for (int v = 0; v < variant_count(); ++v) {
    const double t = plan_estimate_us(v, 1, m, grouped_n(v), k, 0u);
    if (t < best_us) {
      best_us = t;
      best = plan_make(v, 1, m, n_total, k, 0u);
    }
  }
  return best;
}

namespace {
// Bytes-per-K of the distinct X tiles (bm rows each) and W stripes (bn columns
// each) that work ids [a, b) of one split touch in the order of group width g.
double span_cost(uint32_t a, uint32_t b, uint32_t mtiles, uint32_t nstripes, uint32_t g, double bm, double bn) {
  if (a >= b) return 0.0;
  if (g == 0) {
    const uint32_t dm = std::min(b - a, mtiles), ds = (b - 1) / mtiles - a / mtiles + 1;
    return dm * bm + ds * bn;
  }
  const uint32_t gw = mtiles * g;
  double cost = 0.0;
  for (uint32_t grp = a / gw; grp * gw < b; ++grp) {
    const uint32_t gsz = std::min(g, nstripes - grp * g);
    const uint32_t base = grp * gw, lo = std::max(a, base) - base, hi = std::min(b, base + mtiles * gsz) - base;
    if (lo >= hi) continue;
    const uint32_t ds = std::min(hi - lo, gsz), dm = (hi - 1) / gsz - lo / gsz + 1;
    cost += dm * bm + ds * bn;
  }
  return cost;
}

double order_cost(const Plan& p, uint32_t g, double bm, double bn) {
  constexpr uint32_t kXcds = 8, kSlots = 32;  // workgroups per XCD per round (one per CU)
  constexpr uint32_t kRounds = 4;  // rounds counted per XCD: later ones repeat the pattern, and this bounds host time
  const uint32_t per_split = p.mtiles * p.stripes, per = p.grid / kXcds, extra = p.grid % kXcds;
  double cost = 0.0;
  for (uint32_t x = 0; x < kXcds; ++x) {
    const uint32_t start = x * per + std::min(x, extra), count = per + (x < extra ? 1u : 0u);
    for (uint32_t j = 0; j < count && j < kRounds * kSlots; j += kSlots) {
      uint32_t a = start + j;
      const uint32_t b = start + std::min(count, j + kSlots);
      while (a < b) {  // split boundaries: each split reads its own K range
        const uint32_t s = a / per_split, e = std::min(b, (s + 1) * per_split);
        cost += span_cost(a - s * per_split, e - s * per_split, p.mtiles, p.stripes, g, bm, bn);
        a = e;
      }
    }
  }
  return cost;
}

// DH_GEMM_TILE_GROUP=<g>: -1 (unset, or not a number in 0..64) lets the planner choose; 0..64 fixes the order
// (widths past a launch's stripe count act as one group; the cap keeps mtiles · g far from wrapping in the kernel).
int env_tile_group() {
  static const int v = [] {
    const char* e = std::getenv("DH_GEMM_TILE_GROUP");
    if (!e || !*e) return -1;
    char* end = nullptr;
    const long g = std::strtol(e, &end, 10);
    return *end == '\0' && g >= 0 && g <= 64 ? (int)g : -1;
  }();
  return v;
}
}  // namespace

uint32_t plan_order(const Plan& p) {
  if (p.variant == kStreamVariant || p.grid == 0) return 0;
  if (env_tile_group() >= 0) return (uint32_t)env_tile_group();
  if (p.mtiles < 2 || p.stripes < 2) return 0;
  // a forward plans the same few shapes in every layer: the last answers per thread, keyed by what they depend on
  struct Memo {
    int variant = -1;
    uint32_t mtiles = 0, stripes = 0, splits = 0, order = 0;
  };
  thread_local Memo memo[8];
  Memo& mo = memo[(p.mtiles * 31u + p.stripes * 7u + p.splits * 3u + (uint32_t)p.variant) & 7u];
  if (mo.variant == p.variant && mo.mtiles == p.mtiles && mo.stripes == p.stripes && mo.splits == p.splits)
    return mo.order;
  const VariantInfo v = variant_info(p.variant);
  const double bm = v.bm(), bn = v.bn();
  uint32_t best = 0;
  double best_cost = order_cost(p, 0, bm, bn);
  for (uint32_t g : {1u, 2u, 3u, 4u, 6u, 8u}) {
    if (g >= p.stripes) break;
    const double c = order_cost(p, g, bm, bn);
    if (c < best_cost * 0.98) {  // a clear gain only: otherwise keep the M-fastest order
      best_cost = c;
      best = g;
    }
  }
  mo = Memo{p.variant, p.mtiles, p.stripes, p.splits, best};
  return best;
}

}  // namespace dh
