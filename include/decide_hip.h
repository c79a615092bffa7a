/*
 * decide_hip.h — C ABI of the MI355X (gfx950) prefill GEMM path of decide.
 *
 * Every entry point below replaces one method of decide-engine's Metal
 * backend; the reference interface each one stands in for is cited beside it
 * (paths relative to the decide source tree). All entry points:
 *   - take plain device pointers (already offset to the slice they address)
 *     and element counts, never host containers or framework types;
 *   - enqueue onto the caller's HIP stream (`stream`, a hipStream_t; NULL is
 *     the legacy default stream) and never synchronise, so stream order plays
 *     the part of decide's single serial compute encoder;
 *   - return DH_OK or a DH_E* status; on a status other than DH_OK the
 *     calling thread's dh_last_error() holds a one-line message. Contract
 *     violations are reported before anything is launched.
 * The library never allocates or frees caller memory. A context owns only its
 * launch plan and a split-K workspace (device memory it allocates itself).
 * A context is immutable after dh_ctx_create apart from that workspace, which
 * grows under an internal lock; launches on different streams that share a
 * context must not run split-K GEMMs concurrently (they share the workspace).
 */
#ifndef DECIDE_HIP_H
#define DECIDE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define DH_OK 0
#define DH_EINVAL 1   /* a contract violation (shape, stride, alignment, enum) */
#define DH_ELAUNCH 2  /* hipLaunchKernel / hipGetLastError reported an error */
#define DH_ENOMEM 3   /* the split-K workspace could not be allocated */
#define DH_EDEVICE 4  /* no usable gfx950 device, or a HIP runtime call failed */

/* Epilogues: exactly decide's `Epilogue` codes (crates/decide-engine/src/kernels/gemm.rs:15-26). */
#define DH_EPI_STORE_F32 0u  /* y fp32 [M, N] = acc */
#define DH_EPI_STORE_F16 1u  /* y fp16 [M, N] = half(acc) */
#define DH_EPI_ADD_F32 2u    /* y fp32 [M, N] += acc (residual add) */
#define DH_EPI_SWIGLU_F16 3u /* y fp16 [M, N/2] = silu(gate) * up over 16-column gate|up blocks */

/* The gate|up interleave block of DH_EPI_SWIGLU_F16 (decide's SWIGLU_BLOCK, config.rs:31). */
#define DH_SWIGLU_BLOCK 16u

/* dh_ctx_create flags. */
#define DH_GEMM_REFERENCE 1u /* every GEMM runs the simple M-independent kernel (decide's
                                DECIDE_GEMM=baseline, kernels/gemm.rs:56-65) */

typedef struct dh_ctx dh_ctx;

/* One member of a grouped GEMM: Y_i = X · W_iᵀ with its own epilogue. */
typedef struct dh_gemm_member {
  const void* w;   /* fp16 [n, k], row stride ldw (elements) */
  void* y;         /* output, row stride ldy in elements of its output type */
  uint32_t ldw;
  uint32_t ldy;
  uint32_t n;
  uint32_t epi;    /* DH_EPI_* */
} dh_gemm_member;

/* A launch plan as the planner chose it (for tests, tuning and reports). */
typedef struct dh_gemm_plan {
  uint32_t variant;     /* index into the compiled tile-kernel menu */
  uint32_t bm, bn;      /* output tile (rows, columns) */
  uint32_t waves;       /* wavefronts per workgroup */
  uint32_t splits;      /* split-K factor (1 = none) */
  uint32_t workgroups;  /* grid size of the tile kernel */
  uint64_t ws_bytes;    /* split-K workspace the launch needs */
} dh_gemm_plan;

/* --- context (decide: Gemm::new / Gemm::with_impl, kernels/gemm.rs:56-83;
 *     Kernels::new, kernels/mod.rs:53-67) --- */
int dh_ctx_create(uint32_t flags, dh_ctx** out);
void dh_ctx_destroy(dh_ctx* ctx);
/* The calling thread's message for its last failed call ("" if none). */
const char* dh_last_error(void);
/* Library version string. */
const char* dh_version(void);

/* Loads every kernel of the menu and runs each once on a tiny shape, and sizes
 * the split-K workspace for `max_m` rows of the widest planned GEMM, so a timed
 * forward neither loads code nor allocates (decide: Gemm::warm_up, gemm.rs:87-107). */
int dh_warm_up(dh_ctx* ctx, void* stream, uint32_t max_m);
/* Distinct kernels launched through this context so far; after dh_warm_up it
 * must not grow (decide: Gemm::fast_pipelines, gemm.rs:109-113; engine.rs:163-172). */
uint32_t dh_variants_loaded(const dh_ctx* ctx);

/* --- the GEMM operator (decide: Gemm::gemm, kernels/gemm.rs:126-176) ---
 * y = epi(X · Wᵀ): X fp16 [m, k] row stride ldx, W fp16 [n, k] row stride ldw,
 * fp32 accumulation, ldy in elements of y's type. Contract (gemm.rs:140-163):
 * n % 32 == 0, k % 32 == 0, m >= 1, ldx >= k, ldw >= k, ldy >= n (n/2 for
 * SwiGLU), ldx % 8 == 0, ldw % 8 == 0, ldy even, x and w 16-byte aligned, y
 * 8-byte (fp32 outputs) or 4-byte (fp16 outputs) aligned. */
int dh_gemm_nt(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y,
               uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi);

/* Grouped form: every member shares X (m rows, k columns) and is computed in
 * ONE launch. decide has no grouped call; it fuses members by concatenating
 * their weight rows offline (convert.rs:204-245: qkv|z|b|a, q|gate|k|v,
 * gate|up) and calls Gemm::gemm once. This is that launch without the
 * concatenated copy. Same per-member contract as dh_gemm_nt; count in 1..8. */
int dh_gemm_nt_grouped(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, uint32_t m, uint32_t k,
                       const dh_gemm_member* members, uint32_t count);

/* The plan dh_gemm_nt would use (no launch, no device needed; decide:
 * gemm_configs::plan, crates/decide-metal/src/gemm_configs.rs:311-314). */
int dh_gemm_plan_for(const dh_ctx* ctx, uint32_t m, uint32_t n, uint32_t k, uint32_t epi, dh_gemm_plan* out);
/* Forces the next GEMMs on this context to use `variant` and `splits`
 * (variant = UINT32_MAX restores the planner). For tuning sweeps only. */
int dh_gemm_force(dh_ctx* ctx, uint32_t variant, uint32_t splits);
/* Number of compiled tile variants and the geometry of one of them. */
uint32_t dh_gemm_variant_count(void);
int dh_gemm_variant_info(uint32_t variant, uint32_t* bm, uint32_t* bn, uint32_t* waves, uint32_t* wave_cols);

/* --- row gathers (decide: Head::gather_rows_f32 / gather_rows_f16,
 *     kernels/head.rs:28-46; kernels/head.metal:8-28) ---
 * out[i, :] = x[rowmap[i], :] for i < rows, h elements per row, bitwise. The
 * 2-byte form copies any 16-bit rows (fp16 activations, bf16 embedding rows). */
int dh_gather_rows_f32(dh_ctx* ctx, void* stream, const float* x, const uint32_t* rowmap, float* out,
                       uint32_t rows, uint32_t h);
int dh_gather_rows_f16(dh_ctx* ctx, void* stream, const uint16_t* x, const uint32_t* rowmap, uint16_t* out,
                       uint32_t rows, uint32_t h);

/* --- candidate-only LM head (decide: Head::final_head, kernels/head.rs:48-60;
 *     kernels/head.metal:30-59; cpu_ref::final_head, cpu_ref.rs:190-198) ---
 * For each of `rows` fp32 rows of x [rows, hidden]: zero-centred RMSNorm
 * (weight (1 + w), w fp32 [hidden], eps), then the fp32 dot product with the
 * bf16 rows of `table` [vocab, hidden] named by cand[r * max_cand + c] for
 * c < min(ncand[r], max_cand). Writes logits[r * max_cand + c]; entries past
 * ncand[r] are left untouched. decide fixes hidden = 2560 and max_cand = 62;
 * here both are parameters (hidden % 8 == 0, hidden <= 16384, 1 <= max_cand <= 524280).
 * Candidate ids >= vocab are a contract violation the kernel cannot see: the
 * caller validates ids (decide: forward.rs:1494-1537). */
int dh_final_head(dh_ctx* ctx, void* stream, const float* x, const float* w, const uint16_t* table,
                  const uint32_t* cand, const uint32_t* ncand, float* logits, uint32_t rows, uint32_t hidden,
                  uint32_t max_cand, float eps);

/* --- row RMSNorm, fp32 in, fp16 out (decide: Norm::rmsnorm, kernels/norm.rs:26-33;
 *     kernels/rmsnorm.metal:8-30) ---
 * y[r] = half(x[rowmap[r]] * rsqrt(mean(x^2) + eps) * (add_one ? 1 + w : w)).
 * Contract: h <= ld_in and h <= ld_out (norm.rs:27). */
int dh_rmsnorm_rows(dh_ctx* ctx, void* stream, const float* x, const float* w, uint16_t* y,
                    const uint32_t* rowmap, uint32_t rows, uint32_t h, uint32_t ld_in, uint32_t ld_out,
                    uint32_t add_one, float eps);

/* --- synthetic inputs (decide: the random-init role of testutil::uniform,
 *     testutil.rs:4-8, with the Gaussian shapes BASELINE asks for) ---
 * Fills n fp16 values with N(0, std) from a counter-based generator keyed by
 * seed: element i depends only on (seed, i), so fills are reproducible and
 * independent of launch shape. Used to random-initialise weights in place. */
int dh_fill_normal_f16(dh_ctx* ctx, void* stream, uint16_t* out, uint64_t n, uint64_t seed, float std);

/* --- weight layouts (decide: convert.rs:37-62, 74-90), host memory ---
 * Pure permutations / conversions of 16-bit row data, for building the fused
 * operands dh_gemm_nt consumes. */
/* gate, up: [n, k] each → out [2n, k] in blocks of `block` rows: g0 u0 g1 u1 …
 * (n % block == 0). */
int dh_interleave_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint32_t n, uint32_t k,
                          uint32_t block);
/* HF q_proj rows, per head [q_h (head_dim rows); gate_h (head_dim rows)] →
 * [all q rows | all gate rows]. src/out: [heads * 2 * head_dim, k]. */
int dh_deinterleave_q_gate(const uint16_t* src, uint16_t* out, uint32_t heads, uint32_t head_dim, uint32_t k);
/* bf16 bits → fp16 bits, round to nearest even. Returns DH_EINVAL if any finite
 * value overflows fp16 (decide aborts the conversion, convert.rs:168-173);
 * counts[0..3] = {values, subnormal, flushed to zero, overflow} if non-NULL. */
int dh_bf16_to_f16(const uint16_t* src, uint16_t* out, uint64_t n, uint64_t* counts);

#ifdef __cplusplus
}
#endif

#endif /* DECIDE_HIP_H */
