// The dh_model object, shared by the forward host (forward.cpp: weights,
// buffers, one chunk's layers) and the request layer (session.cpp: chunks,
// prefix snapshot, state cache). decide keeps all of this in one struct,
// Forward (crates/decide-engine/src/forward.rs:428-470).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "api_internal.h"

namespace dh_model_impl {

constexpr uint32_t HIDDEN = 2560, NK = 16, DK = 128, NV = 32, DV = 128;
constexpr uint32_t KEY_DIM = NK * DK, VALUE_DIM = NV * DV, CONV_DIM = 2 * KEY_DIM + VALUE_DIM, CONV_K = 4;
constexpr uint32_t LIN_IN_N = CONV_DIM + VALUE_DIM + 2 * NV, LIN_Z = CONV_DIM, LIN_B = CONV_DIM + VALUE_DIM,
                   LIN_A = LIN_B + NV;
constexpr uint32_t NQ = 16, NKV = 4, HEAD_DIM = 256, Q_DIM = NQ * HEAD_DIM, KV_DIM = NKV * HEAD_DIM;
constexpr uint32_t ATT_IN_N = 2 * Q_DIM + 2 * KV_DIM, ATT_K = 2 * Q_DIM, ATT_V = 2 * Q_DIM + KV_DIM;
constexpr uint32_t INTER = 9216, MLP_IN_N = 2 * INTER, ROT_HALF = 32;
constexpr float EPS = 1e-6f;
constexpr uint32_t kCacheRowsMax = 8192;  // decide's MAX_TOKENS (config.rs:35): the K/V cache height
constexpr uint64_t kStateBytes = (uint64_t)NV * DV * DK * 4;  // one linear layer's recurrent state
constexpr uint64_t kConvBytes = (uint64_t)3 * CONV_DIM * 4;   // its last three raw qkv rows
constexpr uint32_t kMaxStateEntries = 4;                      // forward.rs:70 MAX_STATE_ENTRIES
constexpr uint32_t kDefaultStateEntries = 2;                  // forward.rs:72
constexpr uint32_t kStateMarker[4] = {550, 39087, 10485, 198};  // forward.rs:68 STATE_MARKER

inline bool is_full_attention(uint32_t l) { return (l + 1) % 4 == 0; }  // config.rs:39-41

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
  uint32_t lin_index = 0;  // index into the per-linear-layer state buffers
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

// One device allocation with single ownership.
class DevBuf {
 public:
  DevBuf() = default;
  explicit DevBuf(uint64_t bytes) : bytes_(bytes) {
    if (hipMalloc(&ptr_, bytes ? bytes : 16) != hipSuccess) ptr_ = nullptr;
  }
  ~DevBuf() { reset(); }
  DevBuf(DevBuf&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) { o.ptr_ = nullptr; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      reset();
      ptr_ = o.ptr_;
      bytes_ = o.bytes_;
      o.ptr_ = nullptr;
    }
    return *this;
  }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  void reset() {
    if (ptr_) (void)hipFree(ptr_);
    ptr_ = nullptr;
  }
  bool ok() const { return ptr_ != nullptr; }
  uint64_t bytes() const { return bytes_; }
  template <typename T>
  T* as() const {
    return (T*)ptr_;
  }

 private:
  void* ptr_ = nullptr;
  uint64_t bytes_ = 0;
};

// Where chunk 0 of a run reads its conv and recurrent state (forward.rs:183-193).
enum class SourceKind { Zero, Snapshot, State };
struct Source {
  SourceKind kind = SourceKind::Zero;
  size_t entry = 0;  // index into dh_model::states for SourceKind::State
};

// The state after the constant prompt prefix (forward.rs:236-246). The K/V
// rows 0..prefix stay in device memory here (decide keeps them on the CPU).
struct Snapshot {
  std::vector<uint32_t> ids;
  std::vector<DevBuf> state, conv;  // per linear layer
  std::vector<DevBuf> k, v;         // per attention layer: rows 0..ids.size()
};

// The state at the end of a prompt's state section (forward.rs:217-233).
struct StateEntry {
  uint64_t id = 0;
  std::vector<uint32_t> ids;        // the prompt's ids through the state marker
  std::vector<DevBuf> state, conv;  // per linear layer, after `ids`
  std::vector<DevBuf> k, v;         // per attention layer: rows prefix..ids.size(), room for kv_rows
  uint32_t kv_rows = 0;
};

// One chunk of a run (forward.rs:249-269).
struct Chunk {
  uint32_t pos0 = 0, rows = 0;
  uint32_t stage_row = 0;  // the chunk's first row in the run's ids
  bool first = true;       // reads state from the run's Source
  bool keep_state = false; // writes the conv and recurrent state after it
  uint32_t capture = 0;    // the request's state ends after this many of its rows (0: not here)
  uint32_t a0 = 0, n = 0;  // its answers: sorted answers a0 .. a0 + n
};

// Device pointers a run reads and writes.
struct RunArgs {
  const uint32_t* ids = nullptr;       // [run rows] token ids, chunk rows at stage_row
  const uint32_t* ans_rows = nullptr;  // [answers] row of each answer within its chunk
  const uint32_t* ans_pos = nullptr;   // [answers] absolute position of each answer
  const uint32_t* cand = nullptr;      // [answers][max_cand] candidate ids
  const uint32_t* ncand = nullptr;     // [answers]
  float* logits = nullptr;             // [answers][max_cand]
};

enum Route : int32_t { kRouteNone = -1, kRouteSnapshot = 0, kRouteFull = 1, kRouteStateCache = 2 };

}  // namespace dh_model_impl

struct dh_model {
  dh_ctx* ctx = nullptr;
  dh_model_config cfg{};
  std::vector<dh_model_impl::Tensor*> tensors;  // owned
  dh_model_impl::Tensor* embed = nullptr;
  dh_model_impl::Tensor* final_norm = nullptr;
  std::vector<dh_model_impl::Layer> layers;
  uint32_t n_lin = 0, n_att = 0;
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
  std::vector<_Float16*> kc, vc;    // per attention layer [kCacheRows = max_tokens][KV_DIM]
  std::vector<float*> state, conv;  // per linear layer, carried from chunk to chunk
  float* zero_state = nullptr;
  float* zero_conv = nullptr;
  uint32_t* iota = nullptr;
  float* inv_freq = nullptr;
  float* xs = nullptr;
  _Float16* hs = nullptr;
  float* ps = nullptr;
  // a request's device copies (the request layer uploads them)
  uint32_t* req_ids = nullptr;
  uint32_t* req_rows = nullptr;
  uint32_t* req_pos = nullptr;
  uint32_t* req_cand = nullptr;
  uint32_t* req_ncand = nullptr;
  float* req_logits = nullptr;
  std::vector<void*> allocs;
  // the request layer (decide: Forward's fields, forward.rs:440-470)
  uint32_t chunk = 0;  // rows per chunk, 1..max_tokens
  bool prune = true;
  bool has_snapshot = false;
  dh_model_impl::Snapshot snapshot;
  bool prefix_clean = false;
  std::vector<dh_model_impl::StateEntry> states;  // most recently used first
  std::vector<dh_model_impl::StateEntry> free_entries;
  uint32_t state_capacity = dh_model_impl::kDefaultStateEntries;
  std::vector<uint32_t> state_marker;
  int64_t kv_owner = -1;  // id of the entry whose K/V rows prefix..end the caches hold; -1 none
  uint64_t next_entry_id = 0;
  int32_t last_route = dh_model_impl::kRouteNone;
  int64_t last_start = -1;

  ~dh_model();
  void* alloc(uint64_t bytes);
  dh_model_impl::Tensor* add(const std::string& name, uint64_t elems, dh_model_impl::DType dt, float mean, float std);
};

namespace dh_model_impl {
// Embedding, every layer and (for chunks with answers) the head of one chunk
// (decide: encode_chunk, forward.rs:1118-1131). With `capture`, the chunk's
// Chunk::capture row ends the request's state and the linear layers write
// their state there into it.
int encode_chunk(dh_model* m, void* s, const RunArgs& r, const Chunk& ch, Source src, const StateEntry* capture,
                 bool prune);
}  // namespace dh_model_impl
