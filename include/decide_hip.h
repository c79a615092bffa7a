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
 * launch plan and, per stream that uses it, two workspaces (device memory it
 * allocates itself): the split-K partials and the forward kernels' scratch
 * (attention's key pieces and the chunked recurrence's per-chunk matrices).
 * Threads and streams (decide: Gemm is Sync, its pipeline cache behind a
 * mutex, kernels/gemm.rs:46-55, 115-124):
 *   - a context may be shared by host threads and by streams. Its plan is
 *     fixed after dh_ctx_create (dh_gemm_force aside, which is atomic and
 *     meant for tuning), and each stream gets its own workspaces, allocated on
 *     that stream's first call that needs them and grown under an internal
 *     lock, so calls on different streams may overlap;
 *   - a workspace that grows is replaced, and the buffer it replaces stays
 *     allocated until dh_ctx_destroy, so a graph captured earlier
 *     (dh_model_capture) never reads freed memory; a graph keeps using the
 *     workspaces of the stream it was captured on, so its replays must not
 *     overlap other calls on that stream's workspaces;
 *   - a workspace never grows while its stream is being captured: such a call
 *     returns DH_EINVAL (size it first with dh_warm_up or an eager call of the
 *     same size on that stream);
 *   - a stream's workspaces stay with the context until dh_ctx_destroy, and a
 *     stream created later with the same handle reuses them: destroy a stream
 *     only after its work has finished;
 *   - dh_gemm_nt_noalloc's scratch is one array per GPU, shared by every
 *     context on it: its calls must not overlap on one GPU;
 *   - a dh_model (its activations, caches and request state) serves one
 *     request at a time: calls on one model must not overlap.
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
#define DH_DELTA_CHUNKED 2u    /* dh_gated_delta always runs the chunked recurrence */
#define DH_DELTA_SEQUENTIAL 4u /* dh_gated_delta always runs the token-by-token kernel (with neither flag:
                                  chunked for t >= DH_DELTA_CHUNK_MIN_T, token by token below; the choice
                                  decide makes with DECIDE_DELTA, kernels/delta.rs:36-49) */
#define DH_DELTA_CHUNK_MIN_T 320u

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
#define DH_GEMM_STREAM_VARIANT 64u /* dh_gemm_plan.variant of the small-M weight-streaming kernel (M <= 16,
                                      N <= 4096, K % 128 == 0; decide's gemm_nt_small, gemm_fast.metal:429-566): 16 × 32
                                      output tiles, 4 waves, W streamed from HBM straight into registers */
typedef struct dh_gemm_plan {
  uint32_t variant;     /* index into the compiled tile-kernel menu, or DH_GEMM_STREAM_VARIANT */
  uint32_t bm, bn;      /* output tile (rows, columns) */
  uint32_t waves;       /* wavefronts per workgroup */
  uint32_t splits;      /* split-K factor (1 = none) */
  uint32_t workgroups;  /* grid size of the tile kernel */
  uint64_t ws_bytes;    /* split-K workspace the launch needs */
  uint32_t order;       /* work order of the tile kernel: 0 = M tiles fastest; g > 0 = column stripes in groups of
                           g, each group's stripes fastest (chosen per launch so that each XCD's L2 sees a compact
                           block of X rows and W columns); the outputs are the same bits whatever the order. The
                           environment variable DH_GEMM_TILE_GROUP=<g> (0..64), read once per process, fixes it
                           for every launch (for measurements; the library reads no other variable) */
} dh_gemm_plan;

/* --- context (decide: Gemm::new / Gemm::with_impl, kernels/gemm.rs:56-83;
 *     Kernels::new, kernels/mod.rs:53-67) ---
 * Creates a context on the current device (which must be gfx950). Its first
 * creation on a device also takes that device's no-allocation scratch
 * (DH_NOALLOC_SCRATCH_BYTES, shared by every context on the device until the
 * process ends; see dh_gemm_nt_noalloc). Workspaces are per stream (above). */
int dh_ctx_create(uint32_t flags, dh_ctx** out);
void dh_ctx_destroy(dh_ctx* ctx);
/* The calling thread's message for its last failed call ("" if none). */
const char* dh_last_error(void);
/* Library version string. */
const char* dh_version(void);

/* Loads every kernel of the menu and runs each once on a tiny shape, and sizes
 * `stream`'s workspaces so that a timed forward of up to `max_m` rows on that
 * stream neither loads code nor allocates (decide: Gemm::warm_up,
 * gemm.rs:87-107): the split-K workspace for the largest split plan of decide's
 * engine shapes at any M up to max_m, and the forward kernels' workspace, whose
 * attention part is sized even for a GEMM-only context: 8.4 MB at max_m = 1,
 * growing with max_m to 84.5 MB (plus the chunked recurrence's, from
 * DH_DELTA_CHUNK_MIN_T rows). max_m must be in 1..DH_PLAN_MAX_ROWS. */
#define DH_PLAN_MAX_ROWS 65536u
int dh_warm_up(dh_ctx* ctx, void* stream, uint32_t max_m);
/* Distinct kernels launched through this context so far; after dh_warm_up it
 * must not grow (decide: Gemm::fast_pipelines, gemm.rs:109-113; engine.rs:163-172). */
uint32_t dh_variants_loaded(const dh_ctx* ctx);

/* --- the GEMM operator (decide: Gemm::gemm, kernels/gemm.rs:126-176) ---
 * y = epi(X · Wᵀ): X fp16 [m, k] row stride ldx, W fp16 [n, k] row stride ldw,
 * fp32 accumulation, ldy in elements of y's type. Contract (gemm.rs:140-163):
 * n % 32 == 0, k % 32 == 0, m >= 1, ldx >= k, ldw >= k, ldy >= n (n/2 for
 * SwiGLU), ldx % 8 == 0, ldw % 8 == 0, ldy even, x and w 16-byte aligned, y
 * 8-byte (fp32 outputs) or 4-byte (fp16 outputs) aligned, and X's and W's rows
 * each within 4 GiB of their base: ((m - 1)·ldx + k)·2 and ((n - 1)·ldw + k)·2
 * at most 2^32 - 1 bytes (no such limit in decide; its engine shapes are far
 * below it). A DH_GEMM_REFERENCE context checks only the first part, as
 * decide's baseline does (gemm.rs:140-156): shapes and strides, plus each
 * operand aligned to its own element size. */
int dh_gemm_nt(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y,
               uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi);

/* The same GEMM without any allocation: no hipMalloc, hipFree or allocating
 * library call, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid it). decide has no
 * counterpart. Split-K partials go to a device array of the library, file
 * scope, DH_NOALLOC_SCRATCH_BYTES on each GPU, which that GPU holds from the
 * first dh_ctx_create on it until the process ends. The planner picks among
 * plans whose partials fit it; a forced plan (dh_gemm_force) that needs more
 * is refused with DH_EINVAL. Same contract and arguments as dh_gemm_nt; the
 * context's device must be current. Every call on one GPU shares that array
 * and nothing in it needs clearing (each split-K launch writes every partial
 * it reads), but calls that overlap on one GPU (different streams, or
 * different contexts) race on it. */
#define DH_NOALLOC_SCRATCH_BYTES 50331648u /* 48 MiB */
int dh_gemm_nt_noalloc(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y,
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
/* The split-K workspace (bytes) that dh_gemm_nt's planner asks for at its
 * largest over every m in 1..max_m and every epilogue at (n, k), on this
 * context (no device needed; the planner runs once per m, so max_m is capped
 * at DH_PLAN_MAX_ROWS, about 0.3 s of host time per shape there). dh_warm_up
 * holds at least this for decide's engine shapes; a caller with other shapes
 * can size its own calls with it. */
int dh_gemm_ws_need(const dh_ctx* ctx, uint32_t max_m, uint32_t n, uint32_t k, uint64_t* out);
/* Forces the next GEMMs on this context, on every stream, to use `variant` and
 * `splits` (variant = UINT32_MAX restores the planner). For tuning sweeps
 * only: calls already running in other threads see the change at their next
 * plan. */
int dh_gemm_force(dh_ctx* ctx, uint32_t variant, uint32_t splits);
/* Number of compiled tile variants and the geometry of one of them: the tile's
 * rows and columns, its wavefronts (4, or 8 with two per SIMD) and the columns
 * of one wave position (with 8 waves, the two waves of a SIMD split it). */
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

/* --- residual add fused with the norm that follows it (no single counterpart in decide: its forward runs
 *     the projection with the AddF32 epilogue, then rmsnorm over the same rows, forward.rs:1256-1282 with
 *     norm.rs:26-33) ---
 * y += X · Wᵀ (dh_gemm_nt with DH_EPI_ADD_F32, the same contract), then h[r] = half(y[r] * rsqrt(mean(y[r]^2)
 * + eps) * (add_one ? 1 + w : w)) for r < m (dh_rmsnorm_rows with rows r itself, h = n, ld_in = ldy,
 * ld_out = ldh). y and h are bitwise those of the two calls. Where the planner splits K, one kernel sums the
 * partials, adds the residual and norms each row, in place of the split-K reduce and the norm kernel.
 * Contract: as dh_gemm_nt, plus n >= 32 and n <= ldh. */
int dh_gemm_add_rmsnorm(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, float* y,
                        uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, const float* norm_w, uint32_t add_one,
                        float eps, uint16_t* h, uint32_t ldh);

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

/* ======================================================================
 * Forward kernels beside the GEMMs: the non-GEMM steps of decide's hybrid
 * decoder forward (forward.rs:1191-1254). Model constants are decide's
 * (config.rs:4-31): 16 key heads and 32 value heads of 128 dims in the
 * Gated-DeltaNet layers (CONV_DIM 8192 = q 2048 | k 2048 | v 4096), 16 query
 * heads over 4 kv heads of 256 dims in the attention layers.
 * ====================================================================== */

/* decide: Embed::embed (kernels/embed.rs:17; kernels/embed.metal). out fp32
 * [t, h] = the bf16 rows table[ids[i]] widened bitwise. h % 8 == 0, table and
 * out 16-byte aligned. ids < vocab is the caller's check (forward.rs:1494-1537). */
int dh_embed_bf16(dh_ctx* ctx, void* stream, const uint32_t* ids, const uint16_t* table, float* out, uint32_t t,
                  uint32_t h);

/* decide: Conv::conv_silu_l2 (kernels/conv.rs:20-35; cpu_ref::conv_silu_l2,
 * cpu_ref.rs:55-81). Reads the qkv columns 0..8192 of t rows of p (fp32, row
 * stride ldp) and prev, the 3 raw rows before them (fp32 [3, 8192], oldest
 * first); w is fp32 [8192, 4]. Writes fp32 q, k [t, 16, 128] (L2-normed, q also
 * scaled by 128^-1/2) and v [t, 32, 128]. ldp even and >= 8192; p, prev, q, k,
 * v 8-byte and w 16-byte aligned. */
int dh_conv_silu_l2(dh_ctx* ctx, void* stream, const float* p, const float* prev, const float* w, float* q, float* k,
                    float* v, uint32_t t, uint32_t ldp);
/* decide: Conv::conv_state_update (kernels/conv.rs:37-48; cpu_ref.rs:86-95).
 * prev_out [3, 8192] = the raw qkv rows t-3, t-2, t-1 (from prev_in where
 * negative). prev_out may be prev_in. */
int dh_conv_state_update(dh_ctx* ctx, void* stream, const float* p, const float* prev_in, float* prev_out, uint32_t t,
                         uint32_t ldp);

/* decide: Delta::gated_delta (kernels/delta.rs:53-80; cpu_ref::gated_delta,
 * cpu_ref.rs:101-129). fp32 throughout: q, k [t, 16, 128]; v, o [t, 32, 128];
 * a, b rows of stride ldab (value head h at column h); a_log, dt_bias [32];
 * state [32][128 dv][128 dk]. state_in may be state_out; with write_state 0
 * state_out is not written (and may be NULL). t >= 1, ldab >= 32; q, k and the
 * states 16-byte aligned. From t = DH_DELTA_CHUNK_MIN_T on (or always, in a
 * context created with DH_DELTA_CHUNKED) the recurrence runs 64 tokens at a
 * time as fp32 matrix products, in a context workspace that dh_warm_up sizes
 * for max_m tokens (a larger t grows it once); below that (or always, with
 * DH_DELTA_SEQUENTIAL) it runs token by token. */
int dh_gated_delta(dh_ctx* ctx, void* stream, const float* q, const float* k, const float* v, const float* a,
                   const float* b, const float* a_log, const float* dt_bias, const float* state_in, float* state_out,
                   float* o, uint32_t t, uint32_t ldab, uint32_t write_state);

/* decide: Conv::conv_silu_l2 then Delta::gated_delta on its outputs
 * (kernels/conv.rs:20-35, kernels/delta.rs:53-80; forward.rs:1203-1216), in one
 * call on the chunked recurrence: its prep kernel forms q, k and v from p, prev
 * and w itself, with dh_conv_silu_l2's arithmetic, so k and v never go through
 * memory. Results are bitwise those of dh_conv_silu_l2 followed by
 * dh_gated_delta on the chunked path, and q (the only conv output the rest of
 * the recurrence reads) is written as dh_conv_silu_l2 writes it. Arguments as
 * there: p's qkv columns 0..8192 of t rows (row stride ldp, even, >= 8192),
 * prev [3, 8192], w [8192, 4]; a, b rows of stride ldab; q [t, 16, 128] out.
 * Always the chunked path, whatever the context's DH_DELTA_* flags; p and prev
 * 8-byte, w, q and the states 16-byte aligned. */
int dh_conv_gated_delta_chunked(dh_ctx* ctx, void* stream, const float* p, const float* prev, const float* w, float* q,
                                const float* a, const float* b, const float* a_log, const float* dt_bias,
                                const float* state_in, float* state_out, float* o, uint32_t t, uint32_t ldp,
                                uint32_t ldab, uint32_t write_state);

/* decide: GNorm::gated_rmsnorm_silu (kernels/gnorm.rs:19-31; cpu_ref.rs:132-145).
 * y fp16 [t, 4096] = per (row, value head) RMSNorm of o over 128 dims with
 * weight w (fp32 [128], no +1), times silu(z); z rows of stride ldz. */
int dh_gated_rmsnorm_silu(dh_ctx* ctx, void* stream, const float* o, const float* z, const float* w, uint16_t* y,
                          uint32_t t, uint32_t ldz);

/* decide: Rope::q_norm_rope (kernels/rope.rs:25-37; cpu_ref::head_norm_rope,
 * cpu_ref.rs:149-162). For the 16 q heads (column 256 h) of rows of pq (fp32,
 * row stride ldq): zero-centred RMSNorm with qw (fp32 [256], applied as 1 + w),
 * RoPE on dims [0, 64) at position qpos[r] with inv_freq (fp32 [32]); writes
 * fp16 qo [rows, 16, 256]. ldq % 4 == 0; pq, qw 16-byte and qo 8-byte aligned. */
int dh_q_norm_rope(dh_ctx* ctx, void* stream, const float* pq, const float* qw, const float* inv_freq,
                   const uint32_t* qpos, uint16_t* qo, uint32_t rows, uint32_t ldq);
/* decide: Rope::kv_norm_rope (kernels/rope.rs:39-54). Row r at position
 * pos0 + r: the 4 k heads at column kcol, normed and rotated like q, into the
 * fp16 K cache kc [pos][4][256]; the 4 v heads at column vcol copied into the
 * V cache vc. pos0 + rows <= 8192 (decide's MAX_TOKENS cache rows). */
int dh_kv_norm_rope(dh_ctx* ctx, void* stream, const float* pkv, const float* kw, const float* inv_freq, uint16_t* kc,
                    uint16_t* vc, uint32_t rows, uint32_t ldkv, uint32_t kcol, uint32_t vcol, uint32_t pos0);

/* decide: Attn::attention (kernels/attn.rs:80-125; cpu_ref::attention,
 * cpu_ref.rs:167-188). q fp16 [rows, 16, 256]; row r at position qpos[r]
 * attends to cache rows 0..=qpos[r] of kc/vc (fp16 [pos][4][256]); the gate is
 * read from pq (fp32, row stride ldq) at column 4096 + 256 h + d. y fp16
 * [rows, 4096] = softmax(q·kᵀ/16)·v ⊙ σ(gate). rows >= 1, ldq >= 8192 and even;
 * q, kc, vc 16-byte, pq 8-byte, qpos and y 4-byte aligned. Cache rows
 * 0..=max(qpos) must hold finite values. Long query blocks' keys are split
 * across workgroups (cut points at fixed key offsets, sized as if the rows sat
 * at positions 0..rows-1) and merged through the context's forward-kernel
 * workspace, which dh_warm_up sizes. The cut length depends only on `rows`:
 * a row's bits depend on its own query, position and cache rows, and, when its
 * keys span a cut, on the call's row count (rounding only). */
int dh_attention(dh_ctx* ctx, void* stream, const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const float* pq,
                 const uint32_t* qpos, uint16_t* y, uint32_t rows, uint32_t ldq);

/* Random-init fill for every parameter dtype (the role of decide's
 * testutil::uniform, testutil.rs:4-8, with the Gaussians BASELINE asks for):
 * n values N(mean, std) as fp16 (dtype 0), bf16 (1) or fp32 (2), element i a
 * function of (seed, i) only — the generator of dh_fill_normal_f16. */
int dh_fill_normal(dh_ctx* ctx, void* stream, void* out, uint64_t n, uint64_t seed, float mean, float std,
                   uint32_t dtype);

/* ======================================================================
 * The hybrid decoder forward (decide: Forward, crates/decide-engine/src/
 * forward.rs): the host that strings the kernels above into decide's layer
 * order with its buffers and fp16 rounding points, over one stream.
 * dh_model_forward runs the full route from position 0 as one chunk of all
 * T rows, and prunes the last layer (full attention) to the answer rows as
 * decide does (forward.rs:1133-1187); the request calls further down add
 * chunking, the prefix snapshot and the state cache. Weights live in device memory the model owns, named
 * as in decide's decide-weights-v1 index (convert.rs:158-245): "embed" (bf16
 * [vocab, 2560]), "final_norm", "L{l}.in_norm", "L{l}.w_in", "L{l}.w_out",
 * "L{l}.post_norm", "L{l}.w_gu", "L{l}.w_down", and per layer kind
 * "L{l}.conv_w", "L{l}.a_log", "L{l}.dt_bias", "L{l}.gnorm" (Gated-DeltaNet)
 * or "L{l}.q_norm", "L{l}.k_norm" (attention, layers with (l + 1) % 4 == 0).
 * ====================================================================== */
typedef struct dh_model dh_model;

typedef struct dh_model_config {
  uint32_t layers;       /* decoder layers (decide: 32: 36) */
  uint32_t vocab;        /* embedding rows (decide: 248,320; BASELINE: 151,936) */
  uint32_t max_tokens;   /* rows per forward, at most 8192 (decide's MAX_TOKENS) */
  uint32_t max_answers;  /* answer rows per forward (decide: MAX_ANSWERS 16) */
  uint32_t max_cand;     /* candidates per answer row (decide: MAX_CANDIDATES 62) */
} dh_model_config;

/* dh_model_forward flags */
#define DH_FORWARD_NO_PRUNE 1u /* run the last layer over every row (decide: set_prune(false)) */

/* Allocates the weights and activation buffers on the context's device. */
int dh_model_create(dh_ctx* ctx, const dh_model_config* cfg, dh_model** out);
void dh_model_destroy(dh_model* model);
/* Device address, element count and dtype (0 fp16, 1 bf16, 2 fp32) of a
 * weight by its decide-weights-v1 name. */
int dh_model_tensor(const dh_model* model, const char* name, void** ptr, uint64_t* elems, uint32_t* dtype);
/* Name of the model's i-th tensor (i from 0 until it returns NULL). */
const char* dh_model_tensor_name(const dh_model* model, uint32_t i);
/* Fills every tensor of the model from a decide-weights-v1 directory
 * (decide: Weights::open, weights.rs:105-183): `decide-index.json` plus the
 * blobs it lists, tensors at 16 KiB-aligned offsets. Checks decide's format
 * tag, dtypes, alignment and bounds, and that each tensor has the dtype and
 * element count the model holds. Blobs are memory-mapped and each tensor is
 * copied once into device memory. Synchronous. */
int dh_model_load(dh_model* model, const char* dir);
/* Random-initialises every weight on `stream` with dh_fill_normal (BASELINE
 * config 5: fp16 GEMM weights, bf16 embedding, fp32 small parameters). */
int dh_model_init_random(dh_model* model, void* stream, uint64_t seed);
/* One forward over t prompt tokens (device ids [t], each < vocab: the caller
 * validates ids, as decide's engine does, forward.rs:1494-1537), enqueued on
 * `stream`. For the n_ans answer rows (device u32 row indices, which are
 * also their positions) writes logits[r * max_cand + c] for the candidate ids
 * cand[r * max_cand + c], c < ncand[r] (decide: encode_final_head,
 * forward.rs:1296-1306). Does not synchronise. */
int dh_model_forward(dh_model* model, void* stream, const uint32_t* ids, uint32_t t, const uint32_t* ans_rows,
                     uint32_t n_ans, const uint32_t* cand, const uint32_t* ncand, float* logits, uint32_t flags);

/* Whole-forward HIP graph (decide has no counterpart: Metal encodes a command
 * buffer per run; this records the forward's launches once so a serving loop
 * replays them with one launch). Runs one eager forward on `stream` (so every
 * workspace is sized before capture), then captures a second into a graph.
 * Replays read and write the same buffers (ids, answer rows, candidates,
 * logits) with the same T and answer count; their contents may change between
 * replays. `stream` must be a created stream, not the legacy default stream. */
typedef struct dh_graph dh_graph;
int dh_model_capture(dh_model* model, void* stream, const uint32_t* ids, uint32_t t, const uint32_t* ans_rows,
                     uint32_t n_ans, const uint32_t* cand, const uint32_t* ncand, float* logits, uint32_t flags,
                     dh_graph** out);
int dh_graph_launch(dh_graph* graph, void* stream);
void dh_graph_destroy(dh_graph* graph);

/* ======================================================================
 * Requests (decide: Forward::logits, build_snapshot and the state cache,
 * crates/decide-engine/src/forward.rs:641-1116). Host ids and answers; each
 * call enqueues its work on `stream` and waits for it, as decide's do.
 *   - Chunks: a span runs in chunks of at most dh_model_chunk() rows, every
 *     layer of one chunk and then the next, state carried between chunks
 *     (forward.rs:887-915). Default: max_tokens (the whole span in one
 *     chunk); decide's default is CHUNK = 512 (config.rs:36).
 *   - Prefix snapshot: dh_model_build_snapshot runs the constant prompt
 *     prefix from zero state and keeps the state after it.
 *   - Tail truncation: rows after the last answer row never run.
 *   - State cache: an LRU of up to 4 states (default 2) at the end of
 *     prompts' state sections, which end with the state marker (default
 *     decide's STATE_MARKER, forward.rs:68). A request about a new state
 *     captures it on the way; one whose ids start with a cached state's ids
 *     runs from the end of that state.
 * ====================================================================== */
typedef struct dh_answer {
  uint32_t row;          /* absolute logit row (< the request's token count) */
  uint32_t ncand;        /* 1 .. max_cand */
  const uint32_t* cand;  /* host candidate token ids [ncand], each < vocab */
} dh_answer;

/* dh_model_logits flags */
#define DH_LOGITS_FULL 1u /* the full route whatever the ids (decide: logits_full, forward.rs:809-815) */

/* dh_model_last_route routes (decide: Route, forward.rs:196-207) */
#define DH_ROUTE_SNAPSHOT 0
#define DH_ROUTE_FULL 1
#define DH_ROUTE_STATE_CACHE 2

/* Logits of each answer's candidates into logits[i * max_cand + c] for the
 * caller's answer i and c < answers[i].ncand (other entries untouched).
 * Checks decide's contract with its messages (check_ids, sorted_answers,
 * forward.rs:1494-1541) and refuses non-finite logits (forward.rs:876-882).
 * Route: from the snapshot when the ids start with the prefix and every
 * answer row lies after it, from a cached state when the ids also start
 * with that state's ids (the longest such), else the full route
 * (decide: logits, forward.rs:696-735; run_answers, 817-885). */
int dh_model_logits(dh_model* model, void* stream, const uint32_t* ids, uint32_t len, const dh_answer* answers,
                    uint32_t n_answers, float* logits, uint32_t flags);
/* Runs `prefix_ids` (len < max_tokens) from position 0 with zero state and
 * keeps the state after it; replaces any earlier snapshot and empties the
 * state cache (decide: build_snapshot, forward.rs:641-675). */
int dh_model_build_snapshot(dh_model* model, void* stream, const uint32_t* prefix_ids, uint32_t len);
/* The snapshot's prefix length (*has_snapshot 0 before the first build;
 * decide: prefix_len, forward.rs:677-680). */
int dh_model_prefix_len(const dh_model* model, uint32_t* len, int* has_snapshot);
/* How the last dh_model_logits computed its request (DH_ROUTE_*, or -1
 * before the first) and the first position it computed (decide: last_route,
 * last_start, forward.rs:682-694). */
int dh_model_last_route(const dh_model* model, int32_t* route, int64_t* start);
/* Rows per chunk, 1 .. max_tokens (decide: set_chunk, forward.rs:560-566). */
int dh_model_set_chunk(dh_model* model, uint32_t rows);
uint32_t dh_model_chunk(const dh_model* model);
/* Prune the last layer to the answer rows (default on; decide: set_pruning, forward.rs:573-578). */
void dh_model_set_pruning(dh_model* model, int on);
int dh_model_pruning(const dh_model* model);
/* State cache capacity, 0 .. 4 (0 turns it off); shrinking evicts the least
 * recently used entries (decide: set_state_cache, forward.rs:732-743). */
int dh_model_set_state_cache(dh_model* model, uint32_t entries);
uint32_t dh_model_state_cache_capacity(const dh_model* model);
/* Forget every cached state, keeping the buffers for the next captures (forward.rs:745-750). */
void dh_model_forget_states(dh_model* model);
/* The token length of each cached state, most recently used first, into
 * lens[0 .. max); returns the number of entries (decide: cached_states, forward.rs:757-762). */
uint32_t dh_model_cached_states(const dh_model* model, uint32_t* lens, uint32_t max);
/* The ids that end a prompt's state; empties the cache (decide: set_state_marker, forward.rs:764-771). */
int dh_model_set_state_marker(dh_model* model, const uint32_t* marker, uint32_t len);
/* Where a prompt's state ends: one past the first `marker` in
 * ids[prefix .. min(limit, len)]; *found 0 if there is none (decide:
 * state_boundary, forward.rs:1503-1515). Host-only. */
int dh_state_boundary(const uint32_t* ids, uint32_t len, uint32_t prefix, const uint32_t* marker, uint32_t marker_len,
                      uint32_t limit, uint32_t* boundary, int* found);

#ifdef __cplusplus
}
#endif

#endif /* DECIDE_HIP_H */
