// The hybrid decoder forward over the C ABI: decide's Forward
// (crates/decide-engine/src/forward.rs) restated for one MI355X. This file
// holds the weights, the buffers and one chunk's work; session.cpp runs
// requests as chunks against the prefix snapshot and the state cache.
//
// decide's layer order, buffers, fp16 rounding points and last-layer pruning
// (forward.rs:1118-1310) are kept. Chunks default to the whole span (up to
// max_tokens rows): with 288 GB of HBM every activation of a long prompt fits
// many times over, and one chunk gives every GEMM its largest M.
//
// Layer l of a chunk (decide: encode_layer, forward.rs:1189-1268):
//   h = rmsnorm(x, in_norm) fp16
//   Gated-DeltaNet (l + 1) % 4 != 0:
//     p = h·w_inᵀ (qkv | z | b | a, fp32) → conv+SiLU+L2 → q, k, v
//     o = gated_delta(q, k, v, a, b) from the carried state → g = gnorm(o, z) fp16
//   attention:
//     p = h·w_inᵀ (q | gate | k | v) → qo = norm+RoPE(q) fp16; kc, vc caches
//     at the chunk's positions; g = attention(qo, kc, vc, gate) fp16
//   x += g·w_outᵀ;  h = rmsnorm(x, post_norm);  x += SwiGLU(h·w_guᵀ)·w_downᵀ
// The last layer (attention) is pruned to the answer rows when asked, as
// decide does (encode_last_layer_pruned, forward.rs:1133-1187): K/V for
// every row, everything else for the answer rows only; then the candidate
// head (final_head) on the answer rows.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/decide_hip.h"
#include "model_internal.h"

using namespace dh_api;
using namespace dh_model_impl;

dh_model::~dh_model() {
  for (void* a : allocs) (void)hipFree(a);
  for (Tensor* t : tensors) delete t;
}

void* dh_model::alloc(uint64_t bytes) {
  void* ptr = nullptr;
  if (hipMalloc(&ptr, bytes ? bytes : 16) != hipSuccess) return nullptr;
  allocs.push_back(ptr);
  return ptr;
}

Tensor* dh_model::add(const std::string& name, uint64_t elems, DType dt, float mean, float std) {
  Tensor* t = new Tensor();
  t->name = name;
  t->elems = elems;
  t->dtype = dt;
  t->mean = mean;
  t->std = std;
  t->ptr = alloc(t->bytes());
  tensors.push_back(t);
  return t->ptr ? t : nullptr;
}

struct dh_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace {

#define TRY(expr)                \
  do {                           \
    const int rc_ = (expr);      \
    if (rc_ != DH_OK) return rc_; \
  } while (0)

template <typename T>
T* as(void* p) {
  return (T*)p;
}

// h = rmsnorm(x rows) fp16 with (1 + w).
int norm(dh_model* m, void* s, const float* x, const Tensor* w, _Float16* y, uint32_t rows) {
  return dh_rmsnorm_rows(m->ctx, s, x, as<float>(w->ptr), (uint16_t*)y, m->iota, rows, HIDDEN, HIDDEN, HIDDEN, 1, EPS);
}

int gemm(dh_model* m, void* s, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y, uint32_t ldy,
         uint32_t rows, uint32_t n, uint32_t k, uint32_t epi) {
  return dh_gemm_nt(m->ctx, s, x, ldx, w, ldw, y, ldy, rows, n, k, epi);
}

// x += a·wᵀ over `rows` rows (a fp16 [rows, k]), then h = rmsnorm(x) with weight nw when one is given: the
// residual add of a projection and the norm that reads the new x next, as one call (dh_gemm_add_rmsnorm, one
// kernel for both where the projection splits K).
int add_norm(dh_model* m, void* s, const void* a, const Tensor* w, float* x, uint32_t rows, uint32_t k,
             const Tensor* nw, _Float16* h) {
  if (!nw) return gemm(m, s, a, k, w->ptr, k, x, HIDDEN, rows, HIDDEN, k, DH_EPI_ADD_F32);
  return dh_gemm_add_rmsnorm(m->ctx, s, a, k, w->ptr, k, x, HIDDEN, rows, HIDDEN, k, as<float>(nw->ptr), 1, EPS,
                             (uint16_t*)h, HIDDEN);
}

// x += MLP(h) over `rows` rows, h = norm(x, post_norm) on entry (decide: encode_mlp without the ANE split,
// forward.rs:1272-1282); then h = norm(x, next) when the next layer's input norm is given.
int mlp(dh_model* m, void* s, const Layer& L, float* x, _Float16* h, uint32_t rows, const Tensor* next) {
  TRY(gemm(m, s, h, HIDDEN, L.w_gu->ptr, HIDDEN, m->mlp, INTER, rows, MLP_IN_N, HIDDEN, DH_EPI_SWIGLU_F16));
  return add_norm(m, s, m->mlp, L.w_down, x, rows, INTER, next, h);
}

// The (conv, recurrent) state chunk 0 of a run reads for linear layer i (decide: source, forward.rs:1036-1046).
void source_of(dh_model* m, Source src, uint32_t i, const float** conv, const float** state) {
  switch (src.kind) {
    case SourceKind::Zero:
      *conv = m->zero_conv;
      *state = m->zero_state;
      break;
    case SourceKind::Snapshot:
      *conv = m->snapshot.conv[i].as<float>();
      *state = m->snapshot.state[i].as<float>();
      break;
    case SourceKind::State:
      *conv = m->states[src.entry].conv[i].as<float>();
      *state = m->states[src.entry].state[i].as<float>();
      break;
  }
}

// Whether dh_gated_delta runs the chunked recurrence for t rows on this context (its own rule).
bool delta_chunked(const dh_ctx* ctx, uint32_t t) {
  return (ctx->flags & DH_DELTA_CHUNKED) || (!(ctx->flags & DH_DELTA_SEQUENTIAL) && t >= DH_DELTA_CHUNK_MIN_T);
}

// The recurrence over chunk rows from..to, from state_in to state_out (forward.rs:1208-1216).
int delta(dh_model* m, void* s, const Layer& L, uint32_t from, uint32_t to, const float* state_in, float* state_out,
          bool write) {
  const float* pa = m->p + (size_t)from * LIN_IN_N;
  return dh_gated_delta(m->ctx, s, m->q + (size_t)from * KEY_DIM, m->k + (size_t)from * KEY_DIM,
                        m->v + (size_t)from * VALUE_DIM, pa + LIN_A, pa + LIN_B, as<float>(L.a_log->ptr),
                        as<float>(L.dt_bias->ptr), state_in, state_out, m->o + (size_t)from * VALUE_DIM, to - from,
                        LIN_IN_N, write ? 1u : 0u);
}

// Layer L over every row of the chunk (decide: encode_layer, forward.rs:1189-1268). On entry h = norm(x, in_norm)
// (formed by the previous layer's last projection); on exit h = norm(x, next) when `next` is given.
int layer_full(dh_model* m, void* s, const Layer& L, const Chunk& ch, Source src, const StateEntry* entry,
               const Tensor* next) {
  const uint32_t rows = ch.rows;
  if (!L.attn) {
    const uint32_t i = L.lin_index;
    TRY(gemm(m, s, m->h, HIDDEN, L.w_in->ptr, HIDDEN, m->p, LIN_IN_N, rows, LIN_IN_N, HIDDEN, DH_EPI_STORE_F32));
    const float* conv_in = m->conv[i];
    const float* state_in = m->state[i];
    if (ch.first) source_of(m, src, i, &conv_in, &state_in);
    const bool capture = entry && ch.capture;
    if (!capture && delta_chunked(m->ctx, rows)) {
      // conv and the chunked recurrence in one call (the prep kernel forms q, k, v itself); then the conv state,
      // whose in-place update must follow every read of conv_in
      TRY(dh_conv_gated_delta_chunked(m->ctx, s, m->p, conv_in, as<float>(L.conv_w->ptr), m->q, m->p + LIN_A,
                                      m->p + LIN_B, as<float>(L.a_log->ptr), as<float>(L.dt_bias->ptr), state_in,
                                      m->state[i], m->o, rows, LIN_IN_N, LIN_IN_N, ch.keep_state ? 1u : 0u));
      if (ch.keep_state) TRY(dh_conv_state_update(m->ctx, s, m->p, conv_in, m->conv[i], rows, LIN_IN_N));
    } else {
      TRY(dh_conv_silu_l2(m->ctx, s, m->p, conv_in, as<float>(L.conv_w->ptr), m->q, m->k, m->v, rows, LIN_IN_N));
      // the capture's update reads conv_in before the in-place update below may overwrite it
      if (capture)
        TRY(dh_conv_state_update(m->ctx, s, m->p, conv_in, entry->conv[i].as<float>(), ch.capture, LIN_IN_N));
      if (ch.keep_state) TRY(dh_conv_state_update(m->ctx, s, m->p, conv_in, m->conv[i], rows, LIN_IN_N));
      if (capture) {
        // split at the end of the state: the state there goes to the entry, and the
        // rest of the chunk continues from it (fp32 through memory, so exactly)
        float* at = entry->state[i].as<float>();
        TRY(delta(m, s, L, 0, ch.capture, state_in, at, true));
        if (ch.capture < rows)
          TRY(delta(m, s, L, ch.capture, rows, at, m->state[i], ch.keep_state));
        else if (ch.keep_state)
          TRY(hip_status(hipMemcpyAsync(m->state[i], at, kStateBytes, hipMemcpyDeviceToDevice, (hipStream_t)s),
                         "state copy"));
      } else {
        TRY(delta(m, s, L, 0, rows, state_in, m->state[i], ch.keep_state));
      }
    }
    TRY(dh_gated_rmsnorm_silu(m->ctx, s, m->o, m->p + LIN_Z, as<float>(L.gnorm->ptr), (uint16_t*)m->g, rows,
                              LIN_IN_N));
  } else {
    const uint32_t* qpos = m->iota + ch.pos0;
    TRY(gemm(m, s, m->h, HIDDEN, L.w_in->ptr, HIDDEN, m->p, ATT_IN_N, rows, ATT_IN_N, HIDDEN, DH_EPI_STORE_F32));
    TRY(dh_q_norm_rope(m->ctx, s, m->p, as<float>(L.q_norm->ptr), m->inv_freq, qpos, (uint16_t*)m->qo, rows,
                       ATT_IN_N));
    TRY(dh_kv_norm_rope(m->ctx, s, m->p, as<float>(L.k_norm->ptr), m->inv_freq, (uint16_t*)m->kc[L.att_index],
                        (uint16_t*)m->vc[L.att_index], rows, ATT_IN_N, ATT_K, ATT_V, ch.pos0));
    TRY(dh_api::attention_run(m->ctx, s, (const uint16_t*)m->qo, (const uint16_t*)m->kc[L.att_index],
                              (const uint16_t*)m->vc[L.att_index], m->p, qpos, (uint16_t*)m->g, rows, ATT_IN_N,
                              ch.pos0 + rows));
  }
  TRY(add_norm(m, s, m->g, L.w_out, m->x, rows, VALUE_DIM, L.post_norm, m->h));
  return mlp(m, s, L, m->x, m->h, rows, next);
}

// Final norm + candidate logits of the chunk's answers from xs (decide: encode_final_head, forward.rs:1296-1306).
int final_head(dh_model* m, void* s, const RunArgs& r, const Chunk& ch) {
  const uint32_t a0 = ch.a0, mc = m->cfg.max_cand;
  return dh_final_head(m->ctx, s, m->xs + (size_t)a0 * HIDDEN, as<float>(m->final_norm->ptr),
                       (const uint16_t*)m->embed->ptr, r.cand + (size_t)a0 * mc, r.ncand + a0,
                       r.logits + (size_t)a0 * mc, ch.n, HIDDEN, mc, EPS);
}

// The last layer (full attention) pruned to the chunk's answer rows
// (decide: encode_last_layer_pruned, forward.rs:1133-1187). On entry h = norm(x, in_norm) over the chunk's rows.
int layer_pruned(dh_model* m, void* s, const Layer& L, const RunArgs& r, const Chunk& ch) {
  const _Float16* w_in = as<_Float16>(L.w_in->ptr);
  // rows ATT_K.. of w_in are k|v
  TRY(gemm(m, s, m->h, HIDDEN, w_in + (size_t)ATT_K * HIDDEN, HIDDEN, m->p, 2 * KV_DIM, ch.rows, 2 * KV_DIM, HIDDEN,
           DH_EPI_STORE_F32));
  TRY(dh_kv_norm_rope(m->ctx, s, m->p, as<float>(L.k_norm->ptr), m->inv_freq, (uint16_t*)m->kc[L.att_index],
                      (uint16_t*)m->vc[L.att_index], ch.rows, 2 * KV_DIM, 0, KV_DIM, ch.pos0));
  if (ch.n == 0) return ok();
  const uint32_t n = ch.n, a0 = ch.a0;
  const uint32_t* rowmap = r.ans_rows + a0;
  const uint32_t* qpos = r.ans_pos + a0;
  _Float16* hs = m->hs + (size_t)a0 * HIDDEN;
  float* ps = m->ps + (size_t)a0 * ATT_K;
  float* xs = m->xs + (size_t)a0 * HIDDEN;
  TRY(dh_gather_rows_f16(m->ctx, s, (const uint16_t*)m->h, rowmap, (uint16_t*)hs, n, HIDDEN));
  // rows 0..ATT_K of w_in are q|gate
  TRY(gemm(m, s, hs, HIDDEN, w_in, HIDDEN, ps, ATT_K, n, ATT_K, HIDDEN, DH_EPI_STORE_F32));
  TRY(dh_q_norm_rope(m->ctx, s, ps, as<float>(L.q_norm->ptr), m->inv_freq, qpos, (uint16_t*)m->qo, n, ATT_K));
  // the answers sit at positions below the chunk's end
  TRY(dh_api::attention_run(m->ctx, s, (const uint16_t*)m->qo, (const uint16_t*)m->kc[L.att_index],
                            (const uint16_t*)m->vc[L.att_index], ps, qpos, (uint16_t*)m->g, n, ATT_K,
                            ch.pos0 + ch.rows));
  TRY(dh_gather_rows_f32(m->ctx, s, m->x, rowmap, xs, n, HIDDEN));
  TRY(add_norm(m, s, m->g, L.w_out, xs, n, VALUE_DIM, L.post_norm, hs));
  TRY(mlp(m, s, L, xs, hs, n, nullptr));
  return final_head(m, s, r, ch);
}

}  // namespace

int dh_model_impl::encode_chunk(dh_model* m, void* s, const RunArgs& r, const Chunk& ch, Source src,
                                const StateEntry* capture, bool prune) {
  TRY(dh_embed_bf16(m->ctx, s, r.ids + ch.stage_row, (const uint16_t*)m->embed->ptr, m->x, ch.rows, HIDDEN));
  const uint32_t last = m->cfg.layers - 1;
  prune = prune && is_full_attention(last);
  TRY(norm(m, s, m->x, m->layers[0].in_norm, m->h, ch.rows));
  for (uint32_t l = 0; l < last; ++l) TRY(layer_full(m, s, m->layers[l], ch, src, capture, m->layers[l + 1].in_norm));
  if (prune) return layer_pruned(m, s, m->layers[last], r, ch);
  TRY(layer_full(m, s, m->layers[last], ch, src, capture, nullptr));
  if (ch.n == 0) return ok();
  TRY(dh_gather_rows_f32(m->ctx, s, m->x, r.ans_rows + ch.a0, m->xs + (size_t)ch.a0 * HIDDEN, ch.n, HIDDEN));
  return final_head(m, s, r, ch);
}

extern "C" {

int dh_model_create(dh_ctx* ctx, const dh_model_config* cfg, dh_model** out) {
  if (!out) return fail(DH_EINVAL, "model: out is NULL");
  *out = nullptr;
  if (!ctx || !cfg) return fail(DH_EINVAL, "model: null context or config");
  if (cfg->layers < 1) return fail(DH_EINVAL, "model: layers must be at least 1");
  if (cfg->vocab < 1) return fail(DH_EINVAL, "model: vocab must be at least 1");
  if (cfg->max_tokens < 1 || cfg->max_tokens > kCacheRowsMax)
    return fail(DH_EINVAL, "model: max_tokens = %u must be in 1..%u", cfg->max_tokens, kCacheRowsMax);
  if (cfg->max_answers < 1 || cfg->max_answers > cfg->max_tokens)
    return fail(DH_EINVAL, "model: max_answers = %u must be in 1..max_tokens", cfg->max_answers);
  if (cfg->max_cand < 1 || cfg->max_cand > 524280u) return fail(DH_EINVAL, "model: max_cand must be in 1..524280");
  dh_model* m = new dh_model();
  m->ctx = ctx;
  m->cfg = *cfg;
  const uint32_t T = cfg->max_tokens, A = cfg->max_answers;
  bool okay = true;
  auto add = [&](const std::string& name, uint64_t elems, DType dt, float mean, float std) {
    Tensor* t = m->add(name, elems, dt, mean, std);
    okay = okay && t;
    return t;
  };
  // Random-init distributions: fp16 GEMM weights and the
  // bf16 embedding N(0, 0.02); zero-centred norm weights (applied as 1 + w)
  // N(0, 0.02); the gated norm's plain weight N(1, 0.02); conv N(0, 0.3);
  // A_log N(0.5, 0.5) and dt_bias N(0, 0.5), all fp32 (decide keeps them fp32).
  m->embed = add("embed", (uint64_t)cfg->vocab * HIDDEN, BF16, 0.f, 0.02f);
  m->final_norm = add("final_norm", HIDDEN, F32, 0.f, 0.02f);
  uint32_t n_att = 0, n_lin = 0;
  for (uint32_t l = 0; l < cfg->layers && okay; ++l) {
    Layer L;
    const std::string pre = "L" + std::to_string(l) + ".";
    L.attn = is_full_attention(l);
    L.in_norm = add(pre + "in_norm", HIDDEN, F32, 0.f, 0.02f);
    if (L.attn) {
      L.att_index = n_att++;
      L.w_in = add(pre + "w_in", (uint64_t)ATT_IN_N * HIDDEN, F16, 0.f, 0.02f);
      L.q_norm = add(pre + "q_norm", HEAD_DIM, F32, 0.f, 0.02f);
      L.k_norm = add(pre + "k_norm", HEAD_DIM, F32, 0.f, 0.02f);
      L.w_out = add(pre + "w_out", (uint64_t)HIDDEN * Q_DIM, F16, 0.f, 0.02f);
    } else {
      L.lin_index = n_lin++;
      L.w_in = add(pre + "w_in", (uint64_t)LIN_IN_N * HIDDEN, F16, 0.f, 0.02f);
      L.conv_w = add(pre + "conv_w", (uint64_t)CONV_DIM * CONV_K, F32, 0.f, 0.3f);
      L.a_log = add(pre + "a_log", NV, F32, 0.5f, 0.5f);
      L.dt_bias = add(pre + "dt_bias", NV, F32, 0.f, 0.5f);
      L.gnorm = add(pre + "gnorm", DV, F32, 1.f, 0.02f);
      L.w_out = add(pre + "w_out", (uint64_t)HIDDEN * VALUE_DIM, F16, 0.f, 0.02f);
    }
    L.post_norm = add(pre + "post_norm", HIDDEN, F32, 0.f, 0.02f);
    L.w_gu = add(pre + "w_gu", (uint64_t)MLP_IN_N * HIDDEN, F16, 0.f, 0.02f);
    L.w_down = add(pre + "w_down", (uint64_t)HIDDEN * INTER, F16, 0.f, 0.02f);
    m->layers.push_back(L);
  }
  auto buf = [&](uint64_t bytes) {
    void* ptr = m->alloc(bytes);
    okay = okay && ptr;
    return ptr;
  };
  if (okay) {
    m->x = (float*)buf((uint64_t)T * HIDDEN * 4);
    m->h = (_Float16*)buf((uint64_t)T * HIDDEN * 2);
    m->p = (float*)buf((uint64_t)T * LIN_IN_N * 4);
    m->q = (float*)buf((uint64_t)T * KEY_DIM * 4);
    m->k = (float*)buf((uint64_t)T * KEY_DIM * 4);
    m->v = (float*)buf((uint64_t)T * VALUE_DIM * 4);
    m->o = (float*)buf((uint64_t)T * VALUE_DIM * 4);
    m->g = (_Float16*)buf((uint64_t)T * VALUE_DIM * 2);
    m->mlp = (_Float16*)buf((uint64_t)T * INTER * 2);
    m->qo = (_Float16*)buf((uint64_t)T * Q_DIM * 2);
    for (uint32_t a = 0; a < n_att; ++a) {
      m->kc.push_back((_Float16*)buf((uint64_t)T * KV_DIM * 2));
      m->vc.push_back((_Float16*)buf((uint64_t)T * KV_DIM * 2));
    }
    for (uint32_t i = 0; i < n_lin; ++i) {
      m->state.push_back((float*)buf(kStateBytes));
      m->conv.push_back((float*)buf(kConvBytes));
    }
    m->zero_state = (float*)buf(kStateBytes);
    m->zero_conv = (float*)buf(kConvBytes);
    m->iota = (uint32_t*)buf((uint64_t)T * 4);
    m->inv_freq = (float*)buf(ROT_HALF * 4);
    m->xs = (float*)buf((uint64_t)A * HIDDEN * 4);
    m->hs = (_Float16*)buf((uint64_t)A * HIDDEN * 2);
    m->ps = (float*)buf((uint64_t)A * ATT_K * 4);
    m->req_ids = (uint32_t*)buf((uint64_t)T * 4);
    m->req_rows = (uint32_t*)buf((uint64_t)A * 4);
    m->req_pos = (uint32_t*)buf((uint64_t)A * 4);
    m->req_cand = (uint32_t*)buf((uint64_t)A * cfg->max_cand * 4);
    m->req_ncand = (uint32_t*)buf((uint64_t)A * 4);
    m->req_logits = (float*)buf((uint64_t)A * cfg->max_cand * 4);
  }
  m->n_att = n_att;
  m->n_lin = n_lin;
  m->chunk = T;
  m->state_marker.assign(kStateMarker, kStateMarker + 4);
  if (!okay) {
    delete m;
    return fail(DH_ENOMEM, "model: device allocation failed");
  }
  std::vector<uint32_t> iota(T);
  for (uint32_t i = 0; i < T; ++i) iota[i] = i;
  float inv_freq[ROT_HALF];
  for (uint32_t i = 0; i < ROT_HALF; ++i) inv_freq[i] = 1.0f / powf(1e7f, (float)(2 * i) / 64.0f);  // config.rs:43-46
  if (hipMemcpy(m->iota, iota.data(), (size_t)T * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(m->inv_freq, inv_freq, sizeof inv_freq, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemset(m->zero_state, 0, kStateBytes) != hipSuccess || hipMemset(m->zero_conv, 0, kConvBytes) != hipSuccess) {
    delete m;
    return fail(DH_EDEVICE, "model: initialising constant buffers failed");
  }
  *out = m;
  return ok();
}

void dh_model_destroy(dh_model* m) { delete m; }

int dh_model_tensor(const dh_model* m, const char* name, void** ptr, uint64_t* elems, uint32_t* dtype) {
  if (!m || !name) return fail(DH_EINVAL, "model_tensor: null model or name");
  for (const Tensor* t : m->tensors)
    if (t->name == name) {
      if (ptr) *ptr = t->ptr;
      if (elems) *elems = t->elems;
      if (dtype) *dtype = t->dtype;
      return ok();
    }
  return fail(DH_EINVAL, "model_tensor: no tensor named '%s'", name);
}

const char* dh_model_tensor_name(const dh_model* m, uint32_t i) {
  if (!m || i >= m->tensors.size()) return nullptr;
  return m->tensors[i]->name.c_str();
}

int dh_model_init_random(dh_model* m, void* stream, uint64_t seed) {
  if (!m) return fail(DH_EINVAL, "model_init_random: null model");
  for (size_t i = 0; i < m->tensors.size(); ++i) {
    const Tensor* t = m->tensors[i];
    TRY(dh_fill_normal(m->ctx, stream, t->ptr, t->elems, seed + 0x9e3779b97f4a7c15ull * (i + 1), t->mean, t->std,
                       t->dtype));
  }
  return ok();
}

int dh_model_forward(dh_model* m, void* stream, const uint32_t* ids, uint32_t t, const uint32_t* ans_rows,
                     uint32_t n_ans, const uint32_t* cand, const uint32_t* ncand, float* logits, uint32_t flags) {
  if (!m) return fail(DH_EINVAL, "forward: null model");
  if (t < 1 || t > m->cfg.max_tokens)
    return fail(DH_EINVAL, "forward: T = %u must be in 1..%u (the model's max_tokens)", t, m->cfg.max_tokens);
  if (n_ans > m->cfg.max_answers)
    return fail(DH_EINVAL, "forward: %u answers exceed the model's %u", n_ans, m->cfg.max_answers);
  if (!ids || (n_ans && (!ans_rows || !cand || !ncand || !logits))) return fail(DH_EINVAL, "forward: null pointer");
  // the full route as one chunk of all t rows from zero state; answer rows are their positions
  RunArgs r;
  r.ids = ids;
  r.ans_rows = ans_rows;
  r.ans_pos = ans_rows;
  r.cand = cand;
  r.ncand = ncand;
  r.logits = logits;
  Chunk ch;
  ch.rows = t;
  ch.n = n_ans;
  return encode_chunk(m, stream, r, ch, Source{}, nullptr, (flags & DH_FORWARD_NO_PRUNE) == 0);
}

int dh_model_capture(dh_model* m, void* stream, const uint32_t* ids, uint32_t t, const uint32_t* ans_rows,
                     uint32_t n_ans, const uint32_t* cand, const uint32_t* ncand, float* logits, uint32_t flags,
                     dh_graph** out) {
  if (!out) return fail(DH_EINVAL, "model_capture: out is NULL");
  *out = nullptr;
  if (!stream) return fail(DH_EINVAL, "model_capture: capture needs a created stream, not the legacy default stream");
  hipStream_t s = (hipStream_t)stream;
  // One eager forward first: it sizes every workspace, so nothing allocates while capturing.
  TRY(dh_model_forward(m, stream, ids, t, ans_rows, n_ans, cand, ncand, logits, flags));
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail(DH_EDEVICE, "model_capture: %s", hipGetErrorString(e));
  e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return fail(DH_EDEVICE, "model_capture: begin capture: %s", hipGetErrorString(e));
  const int rc = dh_model_forward(m, stream, ids, t, ans_rows, n_ans, cand, ncand, logits, flags);
  hipGraph_t g = nullptr;
  e = hipStreamEndCapture(s, &g);
  if (rc != DH_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess || !g) return fail(DH_EDEVICE, "model_capture: end capture: %s", hipGetErrorString(e));
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return fail(DH_EDEVICE, "model_capture: instantiate: %s", hipGetErrorString(e));
  }
  dh_graph* out_g = new dh_graph();
  out_g->graph = g;
  out_g->exec = ex;
  *out = out_g;
  return ok();
}

int dh_graph_launch(dh_graph* g, void* stream) {
  if (!g || !g->exec) return fail(DH_EINVAL, "graph_launch: null graph");
  return hip_status(hipGraphLaunch(g->exec, (hipStream_t)stream), "graph_launch");
}

void dh_graph_destroy(dh_graph* g) {
  if (!g) return;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
}

}  // extern "C"
