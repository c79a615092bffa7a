// The hybrid decoder forward over the C ABI: decide's Forward
// (crates/decide-engine/src/forward.rs) restated for one MI355X.
//
// decide runs a request as chunks of at most CHUNK = 512 rows (config.rs:36)
// against a prefix snapshot and a state cache. This host keeps decide's layer
// order, buffers, fp16 rounding points and last-layer pruning
// (forward.rs:1125-1310), and runs the full route from position 0 as ONE
// chunk of all T rows: with 288 GB of HBM every activation of a 2,307-token
// prompt fits many times over, and one chunk gives every GEMM its largest M.
//
// Layer l (decide: encode_layer, forward.rs:1197-1268):
//   h = rmsnorm(x, in_norm) fp16
//   Gated-DeltaNet (l + 1) % 4 != 0:
//     p = h·w_inᵀ (qkv | z | b | a, fp32) → conv+SiLU+L2 → q, k, v
//     o = gated_delta(q, k, v, a, b) from zero state → g = gnorm(o, z) fp16
//   attention:
//     p = h·w_inᵀ (q | gate | k | v) → qo = norm+RoPE(q) fp16; kc, vc caches
//     g = attention(qo, kc, vc, gate) fp16
//   x += g·w_outᵀ;  h = rmsnorm(x, post_norm);  x += SwiGLU(h·w_guᵀ)·w_downᵀ
// The last layer (attention) is pruned to the answer rows when asked, as
// decide does (encode_last_layer_pruned, forward.rs:1144-1187): K/V for
// every row, everything else for the answer rows only; then the candidate
// head (final_head) on the answer rows.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/decide_hip.h"
#include "api_internal.h"

using namespace dh_api;

namespace {

constexpr uint32_t HIDDEN = 2560, NK = 16, DK = 128, NV = 32, DV = 128;
constexpr uint32_t KEY_DIM = NK * DK, VALUE_DIM = NV * DV, CONV_DIM = 2 * KEY_DIM + VALUE_DIM, CONV_K = 4;
constexpr uint32_t LIN_IN_N = CONV_DIM + VALUE_DIM + 2 * NV, LIN_Z = CONV_DIM, LIN_B = CONV_DIM + VALUE_DIM,
                   LIN_A = LIN_B + NV;
constexpr uint32_t NQ = 16, NKV = 4, HEAD_DIM = 256, Q_DIM = NQ * HEAD_DIM, KV_DIM = NKV * HEAD_DIM;
constexpr uint32_t ATT_IN_N = 2 * Q_DIM + 2 * KV_DIM, ATT_K = 2 * Q_DIM, ATT_V = 2 * Q_DIM + KV_DIM;
constexpr uint32_t INTER = 9216, MLP_IN_N = 2 * INTER, ROT_HALF = 32;
constexpr float EPS = 1e-6f;
constexpr uint32_t kCacheRowsMax = 8192;  // decide's MAX_TOKENS: the K/V cache height

bool is_full_attention(uint32_t l) { return (l + 1) % 4 == 0; }  // config.rs:39-41

enum DType : uint32_t { F16 = 0, BF16 = 1, F32 = 2 };

struct Tensor {
  std::string name;
  void* ptr = nullptr;
  uint64_t elems = 0;
  DType dtype = F16;
  float mean = 0.f, std = 0.f;  // random-init distribution
  uint64_t bytes() const { return elems * (dtype == F32 ? 4 : 2); }
};

struct Layer {
  bool attn = false;
  uint32_t att_index = 0;  // index into the K/V caches
  Tensor* in_norm = nullptr;
  Tensor* post_norm = nullptr;
  Tensor* w_in = nullptr;
  Tensor* w_out = nullptr;
  Tensor* w_gu = nullptr;
  Tensor* w_down = nullptr;
  Tensor* conv_w = nullptr;
  Tensor* a_log = nullptr;
  Tensor* dt_bias = nullptr;
  Tensor* gnorm = nullptr;
  Tensor* q_norm = nullptr;
  Tensor* k_norm = nullptr;
};

template <typename T>
T* as(void* p) {
  return (T*)p;
}

}  // namespace

struct dh_model {
  dh_ctx* ctx = nullptr;
  dh_model_config cfg{};
  std::vector<Tensor*> tensors;  // owned
  Tensor* embed = nullptr;
  Tensor* final_norm = nullptr;
  std::vector<Layer> layers;
  // activations (decide: Buffers, forward.rs:124-180), sized for cfg.max_tokens rows
  float* x = nullptr;
  _Float16* h = nullptr;
  float* p = nullptr;
  float* q = nullptr;
  float* k = nullptr;
  float* v = nullptr;
  float* o = nullptr;
  _Float16* g = nullptr;
  _Float16* mlp = nullptr;
  _Float16* qo = nullptr;
  std::vector<_Float16*> kc, vc;
  float* zero_state = nullptr;
  float* zero_conv = nullptr;
  uint32_t* iota = nullptr;
  float* inv_freq = nullptr;
  float* xs = nullptr;
  _Float16* hs = nullptr;
  float* ps = nullptr;
  std::vector<void*> allocs;

  ~dh_model() {
    for (void* a : allocs) (void)hipFree(a);
    for (Tensor* t : tensors) delete t;
  }
  void* alloc(uint64_t bytes) {
    void* ptr = nullptr;
    if (hipMalloc(&ptr, bytes ? bytes : 16) != hipSuccess) return nullptr;
    allocs.push_back(ptr);
    return ptr;
  }
  Tensor* add(const std::string& name, uint64_t elems, DType dt, float mean, float std) {
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
};

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

// h = rmsnorm(x rows) fp16 with (1 + w).
int norm(dh_model* m, void* s, const float* x, const Tensor* w, _Float16* y, uint32_t rows) {
  return dh_rmsnorm_rows(m->ctx, s, x, as<float>(w->ptr), (uint16_t*)y, m->iota, rows, HIDDEN, HIDDEN, HIDDEN, 1, EPS);
}

int gemm(dh_model* m, void* s, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y, uint32_t ldy,
         uint32_t rows, uint32_t n, uint32_t k, uint32_t epi) {
  return dh_gemm_nt(m->ctx, s, x, ldx, w, ldw, y, ldy, rows, n, k, epi);
}

// x += MLP(norm(x)) over `rows` rows (decide: encode_mlp without the ANE split, forward.rs:1272-1282).
int mlp(dh_model* m, void* s, const Layer& L, float* x, _Float16* h, uint32_t rows) {
  TRY(norm(m, s, x, L.post_norm, h, rows));
  TRY(gemm(m, s, h, HIDDEN, L.w_gu->ptr, HIDDEN, m->mlp, INTER, rows, MLP_IN_N, HIDDEN, DH_EPI_SWIGLU_F16));
  return gemm(m, s, m->mlp, INTER, L.w_down->ptr, INTER, x, HIDDEN, rows, HIDDEN, INTER, DH_EPI_ADD_F32);
}

int layer_full(dh_model* m, void* s, const Layer& L, uint32_t t) {
  TRY(norm(m, s, m->x, L.in_norm, m->h, t));
  if (!L.attn) {
    TRY(gemm(m, s, m->h, HIDDEN, L.w_in->ptr, HIDDEN, m->p, LIN_IN_N, t, LIN_IN_N, HIDDEN, DH_EPI_STORE_F32));
    TRY(dh_conv_silu_l2(m->ctx, s, m->p, m->zero_conv, as<float>(L.conv_w->ptr), m->q, m->k, m->v, t, LIN_IN_N));
    TRY(dh_gated_delta(m->ctx, s, m->q, m->k, m->v, m->p + LIN_A, m->p + LIN_B, as<float>(L.a_log->ptr),
                       as<float>(L.dt_bias->ptr), m->zero_state, nullptr, m->o, t, LIN_IN_N, 0));
    TRY(dh_gated_rmsnorm_silu(m->ctx, s, m->o, m->p + LIN_Z, as<float>(L.gnorm->ptr), (uint16_t*)m->g, t, LIN_IN_N));
  } else {
    TRY(gemm(m, s, m->h, HIDDEN, L.w_in->ptr, HIDDEN, m->p, ATT_IN_N, t, ATT_IN_N, HIDDEN, DH_EPI_STORE_F32));
    TRY(dh_q_norm_rope(m->ctx, s, m->p, as<float>(L.q_norm->ptr), m->inv_freq, m->iota, (uint16_t*)m->qo, t,
                       ATT_IN_N));
    TRY(dh_kv_norm_rope(m->ctx, s, m->p, as<float>(L.k_norm->ptr), m->inv_freq, (uint16_t*)m->kc[L.att_index],
                        (uint16_t*)m->vc[L.att_index], t, ATT_IN_N, ATT_K, ATT_V, 0));
    TRY(dh_attention(m->ctx, s, (const uint16_t*)m->qo, (const uint16_t*)m->kc[L.att_index],
                     (const uint16_t*)m->vc[L.att_index], m->p, m->iota, (uint16_t*)m->g, t, ATT_IN_N));
  }
  TRY(gemm(m, s, m->g, VALUE_DIM, L.w_out->ptr, VALUE_DIM, m->x, HIDDEN, t, HIDDEN, VALUE_DIM, DH_EPI_ADD_F32));
  return mlp(m, s, L, m->x, m->h, t);
}

// decide: encode_last_layer_pruned (forward.rs:1144-1187).
int layer_pruned(dh_model* m, void* s, const Layer& L, uint32_t t, const uint32_t* ans_rows, uint32_t n) {
  const _Float16* w_in = as<_Float16>(L.w_in->ptr);
  TRY(norm(m, s, m->x, L.in_norm, m->h, t));
  // rows ATT_K.. of w_in are k|v
  TRY(gemm(m, s, m->h, HIDDEN, w_in + (size_t)ATT_K * HIDDEN, HIDDEN, m->p, 2 * KV_DIM, t, 2 * KV_DIM, HIDDEN,
           DH_EPI_STORE_F32));
  TRY(dh_kv_norm_rope(m->ctx, s, m->p, as<float>(L.k_norm->ptr), m->inv_freq, (uint16_t*)m->kc[L.att_index],
                      (uint16_t*)m->vc[L.att_index], t, 2 * KV_DIM, 0, KV_DIM, 0));
  if (n == 0) return ok();
  TRY(dh_gather_rows_f16(m->ctx, s, (const uint16_t*)m->h, ans_rows, (uint16_t*)m->hs, n, HIDDEN));
  // rows 0..ATT_K of w_in are q|gate
  TRY(gemm(m, s, m->hs, HIDDEN, w_in, HIDDEN, m->ps, ATT_K, n, ATT_K, HIDDEN, DH_EPI_STORE_F32));
  TRY(dh_q_norm_rope(m->ctx, s, m->ps, as<float>(L.q_norm->ptr), m->inv_freq, ans_rows, (uint16_t*)m->qo, n, ATT_K));
  TRY(dh_attention(m->ctx, s, (const uint16_t*)m->qo, (const uint16_t*)m->kc[L.att_index],
                   (const uint16_t*)m->vc[L.att_index], m->ps, ans_rows, (uint16_t*)m->g, n, ATT_K));
  TRY(dh_gather_rows_f32(m->ctx, s, m->x, ans_rows, m->xs, n, HIDDEN));
  TRY(gemm(m, s, m->g, VALUE_DIM, L.w_out->ptr, VALUE_DIM, m->xs, HIDDEN, n, HIDDEN, VALUE_DIM, DH_EPI_ADD_F32));
  return mlp(m, s, L, m->xs, m->hs, n);
}

}  // namespace

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
  uint32_t n_att = 0;
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
    m->zero_state = (float*)buf((uint64_t)NV * DV * DK * 4);
    m->zero_conv = (float*)buf((uint64_t)3 * CONV_DIM * 4);
    m->iota = (uint32_t*)buf((uint64_t)T * 4);
    m->inv_freq = (float*)buf(ROT_HALF * 4);
    m->xs = (float*)buf((uint64_t)A * HIDDEN * 4);
    m->hs = (_Float16*)buf((uint64_t)A * HIDDEN * 2);
    m->ps = (float*)buf((uint64_t)A * ATT_K * 4);
  }
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
      hipMemset(m->zero_state, 0, (size_t)NV * DV * DK * 4) != hipSuccess ||
      hipMemset(m->zero_conv, 0, (size_t)3 * CONV_DIM * 4) != hipSuccess) {
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
  const bool prune = (flags & DH_FORWARD_NO_PRUNE) == 0 && is_full_attention(m->cfg.layers - 1);
  void* s = stream;
  TRY(dh_embed_bf16(m->ctx, s, ids, (const uint16_t*)m->embed->ptr, m->x, t, HIDDEN));
  const uint32_t last = m->cfg.layers - 1;
  for (uint32_t l = 0; l < m->cfg.layers; ++l) {
    if (l == last && prune)
      TRY(layer_pruned(m, s, m->layers[l], t, ans_rows, n_ans));
    else
      TRY(layer_full(m, s, m->layers[l], t));
  }
  if (n_ans == 0) return ok();
  if (!prune) TRY(dh_gather_rows_f32(m->ctx, s, m->x, ans_rows, m->xs, n_ans, HIDDEN));
  return dh_final_head(m->ctx, s, m->xs, as<float>(m->final_norm->ptr), (const uint16_t*)m->embed->ptr, cand, ncand,
                       logits, n_ans, HIDDEN, m->cfg.max_cand, EPS);
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
