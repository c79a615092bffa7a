// See plan.h. The model constants are MI355X's public figures: 256 CUs of
// 4 SIMDs at 2.4 GHz, one v_mfma_f32_16x16x32_f16 per 16 clocks per SIMD
// (2.5 PFLOP/s dense fp16), 128 B/clk of LDS and 64 B/clk of L2→CU bandwidth
// per CU, 8 TB/s of HBM.
#include "plan.h"

#include <algorithm>
#include <cmath>
#include <limits>

#include "dh_kernels.h"

namespace dh {

namespace {
constexpr double kClockHz = 2.4e9;
constexpr double kCUs = 256.0;
constexpr double kHbmBps = 8.0e12;
constexpr double kLdsBpc = 128.0;   // LDS bytes per clock per CU
constexpr double kL2Bpc = 64.0;     // L2 → CU bytes per clock per CU
constexpr double kStageOverhead = 1.15;
constexpr double kLaunchUs = 2.0;   // fixed cost of one kernel launch
constexpr double kBlockUs = 0.6;    // workgroup start-up and epilogue
constexpr uint32_t kSplitMenu[] = {1, 2, 3, 4, 6, 8};

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
}  // namespace

Plan plan_make(int variant, uint32_t splits, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  const VariantInfo v = variant_info(variant);
  Plan p{};
  p.variant = variant;
  p.splits = splits;
  const uint32_t stages = ceil_div(k, kBK);
  p.kps = ceil_div(stages, splits) * kBK;
  // Splits that would be empty are dropped.
  p.splits = ceil_div(k, p.kps);
  p.mtiles = ceil_div(m, (uint32_t)v.bm());
  p.stripes = ceil_div(n, (uint32_t)v.bn());
  p.grid = p.mtiles * p.stripes * p.splits;
  p.ws_bytes = p.splits > 1 ? (uint64_t)p.splits * m * n * sizeof(float) : 0;
  p.est_us = plan_estimate_us(variant, p.splits, m, n, k, epi);
  return p;
}

double plan_estimate_us(int variant, uint32_t splits, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  const VariantInfo v = variant_info(variant);
  if (epi == 3u && (v.fn % 2) != 0) return std::numeric_limits<double>::infinity();
  const uint32_t stages = ceil_div(k, kBK);
  if (splits > stages) return std::numeric_limits<double>::infinity();
  const uint32_t st_per_split = ceil_div(stages, splits);
  splits = ceil_div(stages, st_per_split);
  const double mtiles = ceil_div(m, (uint32_t)v.bm()), stripes = ceil_div(n, (uint32_t)v.bn());
  const double blocks = mtiles * stripes * splits;
  // Per-stage clocks of one workgroup (one wave per SIMD).
  const double mfma_clk = 32.0 * v.fm * v.fn;
  const double lds_clk = (1.0 + v.wn) * 16.0 * v.fm * 128.0 / kLdsBpc;
  const double l2_clk = (v.wn * v.fn * 2048.0 + 16.0 * v.fm * 128.0) / kL2Bpc;
  const double stage_clk = std::max(mfma_clk, std::max(lds_clk, l2_clk)) * kStageOverhead;
  const double block_us = st_per_split * stage_clk / kClockHz * 1e6 + kBlockUs;
  const double rounds = std::ceil(blocks / kCUs);
  const double compute_us = rounds * block_us;
  // HBM floor: W once, X once, the output (read too for AddF32), split-K partials twice.
  const double out_b = (epi == 0u || epi == 2u) ? 4.0 : 2.0;
  const double out_cols = epi == 3u ? n / 2.0 : n;
  double bytes = 2.0 * n * k + 2.0 * m * k + out_b * m * out_cols * (epi == 2u ? 2.0 : 1.0);
  double extra_us = 0.0;
  if (splits > 1) {
    const double part = 4.0 * splits * (double)m * n;
    bytes += part;
    extra_us = kLaunchUs + (part + out_b * m * out_cols) / kHbmBps * 1e6;
  }
  const double hbm_us = bytes / kHbmBps * 1e6;
  return std::max(compute_us, hbm_us) + kLaunchUs + extra_us;
}

Plan plan_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t epi, uint64_t max_ws) {
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

Plan plan_grouped(uint32_t m, uint32_t n_total, uint32_t k) {
  Plan best{};
  best.est_us = std::numeric_limits<double>::infinity();
  best.variant = -1;
  for (int v = 0; v < variant_count(); ++v) {
    const double t = plan_estimate_us(v, 1, m, n_total, k, 0u);
    if (t < best.est_us) best = plan_make(v, 1, m, n_total, k, 0u);
  }
  return best;
}

}  // namespace dh
