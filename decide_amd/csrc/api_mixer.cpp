// C ABI of the non-GEMM forward kernels (include/decide_hip.h, "forward
// kernels"). Each entry restates the asserts of the decide-engine wrapper it
// replaces and returns DH_EINVAL with a message instead of panicking; nothing
// is launched after a failed check.
#include <cmath>

#include "api_internal.h"
#include "dh_kernels.h"

using namespace dh_api;

namespace {
constexpr uint32_t kConvDim = 8192, kValueDim = 4096, kNV = 32, kQDim = 4096, kMaxTokens = 8192;

bool misaligned(const void* p, uintptr_t a) { return p && !aligned(p, a); }
}  // namespace

namespace dh_api {

int attention_run(dh_ctx* ctx, void* stream, const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                  const float* pq, const uint32_t* qpos, uint16_t* y, uint32_t rows, uint32_t ldq, uint32_t npos) {
  if (rows < 1) return fail(DH_EINVAL, "attention: rows must be at least 1");
  if (ldq < 2 * kQDim) return fail(DH_EINVAL, "attention: ldq = %u must cover the gate columns", ldq);
  if (misaligned(q, 16) || misaligned(kc, 16) || misaligned(vc, 16))
    return fail(DH_EINVAL, "attention: q, kc and vc must be 16-byte aligned");
  if (misaligned(pq, 8) || ldq % 2 != 0)
    return fail(DH_EINVAL, "attention: pq must be 8-byte aligned and ldq = %u even", ldq);
  if (misaligned(qpos, 4) || misaligned(y, 4)) return fail(DH_EINVAL, "attention: qpos and y must be 4-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "attention: null context");
  if (!q || !kc || !vc || !pq || !qpos || !y) return fail(DH_EINVAL, "attention: null pointer");
  const dh::AttnSplit sp = dh::attention_split(rows, npos, ctx->cus);
  const uint64_t ws = dh::attention_ws_bytes(rows, sp);
  float* aux = nullptr;
  if (ws) {  // allocates only past what dh_warm_up (or an earlier call) sized this stream's workspace for
    const int rc = ensure_aux(ctx, (hipStream_t)stream, ws, &aux);
    if (rc != DH_OK) return rc;
    mark(ctx, kKidAttnCombine);
  }
  mark(ctx, kKidAttn);
  return hip_status(dh::launch_attention((const _Float16*)q, (const _Float16*)kc, (const _Float16*)vc, pq, qpos,
                                         (_Float16*)y, aux, rows, ldq, sp, (hipStream_t)stream),
                    "attention");
}

}  // namespace dh_api

extern "C" {

int dh_embed_bf16(dh_ctx* ctx, void* stream, const uint32_t* ids, const uint16_t* table, float* out, uint32_t t,
                  uint32_t h) {
  if (h == 0 || h % 8 != 0) return fail(DH_EINVAL, "embed: H = %u must be a positive multiple of 8", h);
  if (misaligned(table, 16) || misaligned(out, 16))
    return fail(DH_EINVAL, "embed: table and out must be 16-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "embed: null context");
  if (t && (!ids || !table || !out)) return fail(DH_EINVAL, "embed: null pointer");
  mark(ctx, kKidEmbed);
  return hip_status(dh::launch_embed_bf16(ids, table, out, t, h, (hipStream_t)stream), "embed_bf16");
}

int dh_conv_silu_l2(dh_ctx* ctx, void* stream, const float* p, const float* prev, const float* w, float* q, float* k,
                    float* v, uint32_t t, uint32_t ldp) {
  if (ldp < kConvDim || ldp % 2 != 0)
    return fail(DH_EINVAL, "conv: ldp = %u must be even and cover the %u qkv columns", ldp, kConvDim);
  if (misaligned(p, 8) || misaligned(prev, 8) || misaligned(q, 8) || misaligned(k, 8) || misaligned(v, 8) ||
      misaligned(w, 16))
    return fail(DH_EINVAL, "conv: p/prev/q/k/v must be 8-byte and w 16-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "conv: null context");
  if (t && (!p || !prev || !w || !q || !k || !v)) return fail(DH_EINVAL, "conv: null pointer");
  mark(ctx, kKidConv);
  return hip_status(dh::launch_conv_silu_l2(p, prev, w, q, k, v, t, ldp, (hipStream_t)stream), "conv_silu_l2");
}

int dh_conv_state_update(dh_ctx* ctx, void* stream, const float* p, const float* prev_in, float* prev_out, uint32_t t,
                         uint32_t ldp) {
  if (ldp < kConvDim) return fail(DH_EINVAL, "conv_state_update: ldp = %u must cover the %u qkv columns", ldp, kConvDim);
  if (!ctx) return fail(DH_EINVAL, "conv_state_update: null context");
  if (!prev_in || !prev_out || (t && !p)) return fail(DH_EINVAL, "conv_state_update: null pointer");
  mark(ctx, kKidConvState);
  return hip_status(dh::launch_conv_state_update(p, prev_in, prev_out, t, ldp, (hipStream_t)stream),
                    "conv_state_update");
}

int dh_gated_delta(dh_ctx* ctx, void* stream, const float* q, const float* k, const float* v, const float* a,
                   const float* b, const float* a_log, const float* dt_bias, const float* state_in, float* state_out,
                   float* o, uint32_t t, uint32_t ldab, uint32_t write_state) {
  if (t < 1) return fail(DH_EINVAL, "delta: T must be at least 1");
  if (ldab < kNV) return fail(DH_EINVAL, "delta: ldab = %u must cover the %u value heads", ldab, kNV);
  const void* ptrs[] = {q, k, v, a, b, a_log, dt_bias, state_in, state_out, o};
  const char* names[] = {"q", "k", "v", "a", "b", "a_log", "dt_bias", "state_in", "state_out", "o"};
  for (int i = 0; i < 10; ++i) {
    if (misaligned(ptrs[i], 4)) return fail(DH_EINVAL, "delta: %s address must be a multiple of 4", names[i]);
    if (!ptrs[i] && !(i == 8 && !write_state)) return fail(DH_EINVAL, "delta: %s is null", names[i]);
  }
  if (misaligned(q, 16) || misaligned(k, 16) || misaligned(state_in, 16) || misaligned(state_out, 16))
    return fail(DH_EINVAL, "delta: q, k and the states must be 16-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "delta: null context");
  const bool chunked = (ctx->flags & DH_DELTA_CHUNKED) ||
                       (!(ctx->flags & DH_DELTA_SEQUENTIAL) && t >= DH_DELTA_CHUNK_MIN_T);
  if (!chunked) {
    mark(ctx, kKidDelta);
    return hip_status(dh::launch_gated_delta(q, k, v, a, b, a_log, dt_bias, state_in, state_out, o, t, ldab,
                                             write_state != 0, (hipStream_t)stream),
                      "gated_delta");
  }
  // allocates only when T exceeds what dh_warm_up (or an earlier call) sized this stream's workspace for
  float* aux = nullptr;
  const int rc = ensure_aux(ctx, (hipStream_t)stream, dh::delta_chunk_ws_floats(t) * sizeof(float), &aux);
  if (rc != DH_OK) return rc;
  mark(ctx, kKidDeltaChunk);
  return hip_status(dh::launch_gated_delta_chunked(q, k, v, a, b, a_log, dt_bias, state_in, state_out, o, aux, t,
                                                   ldab, write_state != 0, (hipStream_t)stream),
                    "gated_delta (chunked)");
}

int dh_conv_gated_delta_chunked(dh_ctx* ctx, void* stream, const float* p, const float* prev, const float* w, float* q,
                                const float* a, const float* b, const float* a_log, const float* dt_bias,
                                const float* state_in, float* state_out, float* o, uint32_t t, uint32_t ldp,
                                uint32_t ldab, uint32_t write_state) {
  if (t < 1) return fail(DH_EINVAL, "conv_delta: T must be at least 1");
  if (ldp < kConvDim || ldp % 2 != 0)
    return fail(DH_EINVAL, "conv_delta: ldp = %u must be even and cover the %u qkv columns", ldp, kConvDim);
  if (ldab < kNV) return fail(DH_EINVAL, "conv_delta: ldab = %u must cover the %u value heads", ldab, kNV);
  const void* ptrs[] = {p, prev, w, q, a, b, a_log, dt_bias, state_in, state_out, o};
  const char* names[] = {"p", "prev", "w", "q", "a", "b", "a_log", "dt_bias", "state_in", "state_out", "o"};
  for (int i = 0; i < 11; ++i) {
    if (misaligned(ptrs[i], 4)) return fail(DH_EINVAL, "conv_delta: %s address must be a multiple of 4", names[i]);
    if (!ptrs[i] && !(i == 9 && !write_state)) return fail(DH_EINVAL, "conv_delta: %s is null", names[i]);
  }
  if (misaligned(p, 8) || misaligned(prev, 8) || misaligned(w, 16) || misaligned(q, 16) || misaligned(state_in, 16) ||
      misaligned(state_out, 16))
    return fail(DH_EINVAL, "conv_delta: p and prev must be 8-byte, w, q and the states 16-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "conv_delta: null context");
  // allocates only when T exceeds what dh_warm_up (or an earlier call) sized this stream's workspace for
  float* aux = nullptr;
  const int rc = ensure_aux(ctx, (hipStream_t)stream, dh::delta_chunk_ws_floats(t) * sizeof(float), &aux);
  if (rc != DH_OK) return rc;
  mark(ctx, kKidConvDelta);
  return hip_status(dh::launch_conv_gated_delta_chunked(p, prev, w, ldp, q, a, b, ldab, a_log, dt_bias, state_in,
                                                        state_out, o, aux, t, write_state != 0,
                                                        (hipStream_t)stream),
                    "conv + gated_delta (chunked)");
}

int dh_gated_rmsnorm_silu(dh_ctx* ctx, void* stream, const float* o, const float* z, const float* w, uint16_t* y,
                          uint32_t t, uint32_t ldz) {
  if (ldz < kValueDim || ldz % 2 != 0)
    return fail(DH_EINVAL, "gnorm: ldz = %u must be even and cover the %u z columns", ldz, kValueDim);
  if (misaligned(o, 8) || misaligned(z, 8) || misaligned(w, 8) || misaligned(y, 4))
    return fail(DH_EINVAL, "gnorm: o, z, w must be 8-byte and y 4-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "gnorm: null context");
  if (t && (!o || !z || !w || !y)) return fail(DH_EINVAL, "gnorm: null pointer");
  mark(ctx, kKidGNorm);
  return hip_status(dh::launch_gated_rmsnorm_silu(o, z, w, (_Float16*)y, t, ldz, (hipStream_t)stream),
                    "gated_rmsnorm_silu");
}

int dh_q_norm_rope(dh_ctx* ctx, void* stream, const float* pq, const float* qw, const float* inv_freq,
                   const uint32_t* qpos, uint16_t* qo, uint32_t rows, uint32_t ldq) {
  if (ldq < kQDim || ldq % 4 != 0)
    return fail(DH_EINVAL, "q_norm_rope: ldq = %u must be a multiple of 4 covering the %u q columns", ldq, kQDim);
  if (misaligned(pq, 16) || misaligned(qw, 16) || misaligned(qo, 8))
    return fail(DH_EINVAL, "q_norm_rope: pq and qw must be 16-byte and qo 8-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "q_norm_rope: null context");
  if (rows && (!pq || !qw || !inv_freq || !qpos || !qo)) return fail(DH_EINVAL, "q_norm_rope: null pointer");
  mark(ctx, kKidQRope);
  return hip_status(dh::launch_q_norm_rope(pq, qw, inv_freq, qpos, (_Float16*)qo, rows, ldq, (hipStream_t)stream),
                    "q_norm_rope");
}

int dh_kv_norm_rope(dh_ctx* ctx, void* stream, const float* pkv, const float* kw, const float* inv_freq, uint16_t* kc,
                    uint16_t* vc, uint32_t rows, uint32_t ldkv, uint32_t kcol, uint32_t vcol, uint32_t pos0) {
  if ((uint64_t)pos0 + rows > kMaxTokens)
    return fail(DH_EINVAL, "kv_norm_rope: positions %u..%u overrun the %u-row cache", pos0, pos0 + rows, kMaxTokens);
  if (ldkv % 4 != 0 || kcol % 4 != 0 || vcol % 4 != 0 || kcol + 1024 > ldkv || vcol + 1024 > ldkv)
    return fail(DH_EINVAL, "kv_norm_rope: ldkv = %u, kcol = %u, vcol = %u must be multiples of 4 with both 1024-column "
                "groups inside a row", ldkv, kcol, vcol);
  if (misaligned(pkv, 16) || misaligned(kw, 16) || misaligned(kc, 8) || misaligned(vc, 8))
    return fail(DH_EINVAL, "kv_norm_rope: pkv and kw must be 16-byte and the caches 8-byte aligned");
  if (!ctx) return fail(DH_EINVAL, "kv_norm_rope: null context");
  if (rows && (!pkv || !kw || !inv_freq || !kc || !vc)) return fail(DH_EINVAL, "kv_norm_rope: null pointer");
  mark(ctx, kKidKVRope);
  return hip_status(dh::launch_kv_norm_rope(pkv, kw, inv_freq, (_Float16*)kc, (_Float16*)vc, rows, ldkv, kcol, vcol,
                                            pos0, (hipStream_t)stream),
                    "kv_norm_rope");
}

int dh_attention(dh_ctx* ctx, void* stream, const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const float* pq,
                 const uint32_t* qpos, uint16_t* y, uint32_t rows, uint32_t ldq) {
  // decide's interface carries no cache length: the key pieces are sized as if the rows were a prompt's first
  // `rows` positions (any positions stay correct; only the load balance assumes it)
  return attention_run(ctx, stream, q, kc, vc, pq, qpos, y, rows, ldq, rows);
}

int dh_fill_normal(dh_ctx* ctx, void* stream, void* out, uint64_t n, uint64_t seed, float mean, float std,
                   uint32_t dtype) {
  if (dtype > 2) return fail(DH_EINVAL, "fill_normal: dtype %u is not one of 0 (fp16), 1 (bf16), 2 (fp32)", dtype);
  if (!(std >= 0.0f) || !std::isfinite(std) || !std::isfinite(mean))
    return fail(DH_EINVAL, "fill_normal: mean and std must be finite, std >= 0");
  if (misaligned(out, dtype == 2 ? 4 : 2)) return fail(DH_EINVAL, "fill_normal: out is misaligned for its dtype");
  if (!ctx) return fail(DH_EINVAL, "fill_normal: null context");
  if (n && !out) return fail(DH_EINVAL, "fill_normal: null pointer");
  mark(ctx, kKidFillAny);
  return hip_status(dh::launch_fill_normal(out, n, seed, mean, std, dtype, (hipStream_t)stream), "fill_normal");
}

}  // extern "C"
