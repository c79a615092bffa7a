// Requests over the forward host: decide's request layer (Forward::logits,
// build_snapshot and the state cache, crates/decide-engine/src/forward.rs:
// 641-1116) restated on HIP.
//
//   * Chunks. A span of positions start..end runs in chunks of at most
//     `chunk` rows, all layers of one chunk and then the next; each linear
//     layer carries its conv and recurrent state from chunk to chunk, each
//     attention layer writes the chunk's K/V rows at their positions before
//     attending. Chunk 0 reads its state from a Source: zeros, the prefix
//     snapshot or a state-cache entry.
//   * Prefix snapshot. build_snapshot runs the constant prompt prefix once
//     and keeps the state after it; a request whose ids start with the
//     prefix (and whose answers lie after it) runs from there.
//   * Tail truncation. Rows after the last answer row never run.
//   * State cache. A small LRU of the states at the end of prompts' state
//     sections (ending with the state marker). A request about a new state
//     captures it on the way (its chunk splits only the recurrence there);
//     a request whose ids start with a cached state's ids runs from the end
//     of that state, putting its K/V rows back first if another run has
//     overwritten them.
// The snapshot's and the entries' K/V rows stay in device memory (decide
// keeps the snapshot's on the CPU); copies between them and the caches are
// device-to-device on the request's stream. Every call here is synchronous,
// as decide's are (it waits for the command buffer).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/decide_hip.h"
#include "model_internal.h"

using namespace dh_api;
using namespace dh_model_impl;

namespace {

#define TRY(expr)                \
  do {                           \
    const int rc_ = (expr);      \
    if (rc_ != DH_OK) return rc_; \
  } while (0)

struct Answer {
  uint32_t index, row, ncand;
  const uint32_t* cand;
};

// decide: check_ids (forward.rs:1494-1501).
int check_ids(const dh_model* m, const uint32_t* ids, uint32_t len) {
  if (len == 0) return fail(DH_EINVAL, "no input tokens");
  if (!ids) return fail(DH_EINVAL, "null ids");
  if (len > m->cfg.max_tokens)
    return fail(DH_EINVAL, "%u input tokens; the model takes at most %u", len, m->cfg.max_tokens);
  for (uint32_t i = 0; i < len; ++i)
    if (ids[i] >= m->cfg.vocab)
      return fail(DH_EINVAL, "token id %u is outside the %u-token vocabulary", ids[i], m->cfg.vocab);
  return ok();
}

// decide: sorted_answers (forward.rs:1517-1541): validated, sorted by (row, index).
int sorted_answers(const dh_model* m, uint32_t len, const dh_answer* answers, uint32_t n, std::vector<Answer>& out) {
  if (n < 1 || n > m->cfg.max_answers)
    return fail(DH_EINVAL, "%u answers; a request has 1 to %u", n, m->cfg.max_answers);
  if (!answers) return fail(DH_EINVAL, "null answers");
  out.clear();
  for (uint32_t i = 0; i < n; ++i) {
    const dh_answer& a = answers[i];
    if (a.row >= len) return fail(DH_EINVAL, "answer %u: logit row %u is past the %u-token input", i, a.row, len);
    if (a.ncand < 1 || a.ncand > m->cfg.max_cand)
      return fail(DH_EINVAL, "answer %u: %u candidates; a field has 1 to %u", i, a.ncand, m->cfg.max_cand);
    if (!a.cand) return fail(DH_EINVAL, "answer %u: null candidates", i);
    for (uint32_t c = 0; c < a.ncand; ++c)
      if (a.cand[c] >= m->cfg.vocab)
        return fail(DH_EINVAL, "answer %u: candidate %u is outside the %u-token vocabulary", i, a.cand[c],
                    m->cfg.vocab);
    out.push_back(Answer{i, a.row, a.ncand, a.cand});
  }
  std::stable_sort(out.begin(), out.end(), [](const Answer& x, const Answer& y) {
    return x.row != y.row ? x.row < y.row : x.index < y.index;
  });
  return ok();
}

// decide: state_boundary (forward.rs:1503-1515). One past the first `marker`
// in ids[prefix .. min(limit, len)], or false.
bool state_boundary(const uint32_t* ids, uint32_t len, uint32_t prefix, const uint32_t* marker, uint32_t mlen,
                    uint32_t limit, uint32_t* boundary) {
  const uint32_t hi = std::min(limit, len);
  if (mlen == 0 || prefix > hi || hi - prefix < mlen) return false;
  for (uint32_t i = prefix; i + mlen <= hi; ++i)
    if (std::equal(marker, marker + mlen, ids + i)) {
      *boundary = i + mlen;
      return true;
    }
  return false;
}

bool starts_with(const uint32_t* ids, uint32_t len, const std::vector<uint32_t>& pre) {
  return pre.size() <= len && std::equal(pre.begin(), pre.end(), ids);
}

// decide: chunks (forward.rs:887-915).
std::vector<Chunk> make_chunks(uint32_t chunk, uint32_t start, uint32_t end, bool keep_final_state,
                               const std::vector<Answer>& answers) {
  std::vector<Chunk> out;
  uint32_t pos0 = start, a = 0;
  while (pos0 < end) {
    const uint32_t rows = std::min(chunk, end - pos0);
    const bool last = pos0 + rows == end;
    const uint32_t a0 = a;
    while (a < answers.size() && answers[a].row < pos0 + rows) ++a;
    Chunk ch;
    ch.pos0 = pos0;
    ch.rows = rows;
    ch.stage_row = pos0 - start;
    ch.first = pos0 == start;
    ch.keep_state = !last || keep_final_state;
    ch.a0 = a0;
    ch.n = a - a0;
    out.push_back(ch);
    pos0 += rows;
  }
  return out;
}

hipStream_t hs(void* s) { return (hipStream_t)s; }

int copy(void* dst, const void* src, uint64_t bytes, hipMemcpyKind kind, void* s, const char* what) {
  if (bytes == 0) return ok();
  return hip_status(hipMemcpyAsync(dst, src, bytes, kind, hs(s)), what);
}

int sync(void* s) { return hip_status(hipStreamSynchronize(hs(s)), "stream synchronize"); }

// Device buffers for per-layer state: one per linear layer of each kind.
bool alloc_states(const dh_model* m, std::vector<DevBuf>& state, std::vector<DevBuf>& conv) {
  state.clear();
  conv.clear();
  for (uint32_t i = 0; i < m->n_lin; ++i) {
    state.emplace_back(kStateBytes);
    conv.emplace_back(kConvBytes);
    if (!state.back().ok() || !conv.back().ok()) return false;
  }
  return true;
}

bool alloc_kv(const dh_model* m, uint32_t rows, std::vector<DevBuf>& k, std::vector<DevBuf>& v) {
  k.clear();
  v.clear();
  for (uint32_t a = 0; a < m->n_att; ++a) {
    k.emplace_back((uint64_t)rows * KV_DIM * 2);
    v.emplace_back((uint64_t)rows * KV_DIM * 2);
    if (!k.back().ok() || !v.back().ok()) return false;
  }
  return true;
}

// decide: forget_states (forward.rs:745-750).
void forget_states(dh_model* m) {
  for (StateEntry& e : m->states) m->free_entries.push_back(std::move(e));
  m->states.clear();
  m->kv_owner = -1;
}

// Copy an entry's K/V rows (positions prefix .. entry end) from the caches
// into the entry, or back (decide: encode_state_rows, forward.rs:1082-1098).
int state_rows(dh_model* m, void* s, const StateEntry& e, uint32_t prefix, bool to_entry) {
  const uint64_t bytes = (uint64_t)(e.ids.size() - prefix) * KV_DIM * 2;
  for (uint32_t a = 0; a < m->n_att; ++a) {
    _Float16* kc = m->kc[a] + (size_t)prefix * KV_DIM;
    _Float16* vc = m->vc[a] + (size_t)prefix * KV_DIM;
    if (to_entry) {
      TRY(copy(e.k[a].as<void>(), kc, bytes, hipMemcpyDeviceToDevice, s, "state K rows"));
      TRY(copy(e.v[a].as<void>(), vc, bytes, hipMemcpyDeviceToDevice, s, "state V rows"));
    } else {
      TRY(copy(kc, e.k[a].as<void>(), bytes, hipMemcpyDeviceToDevice, s, "state K rows"));
      TRY(copy(vc, e.v[a].as<void>(), bytes, hipMemcpyDeviceToDevice, s, "state V rows"));
    }
  }
  return ok();
}

// Put the snapshot's K/V rows back into rows 0..prefix of the caches (decide: restore_prefix, forward.rs:1026-1033).
int restore_prefix(dh_model* m, void* s) {
  const uint64_t bytes = (uint64_t)m->snapshot.ids.size() * KV_DIM * 2;
  for (uint32_t a = 0; a < m->n_att; ++a) {
    TRY(copy(m->kc[a], m->snapshot.k[a].as<void>(), bytes, hipMemcpyDeviceToDevice, s, "prefix K rows"));
    TRY(copy(m->vc[a], m->snapshot.v[a].as<void>(), bytes, hipMemcpyDeviceToDevice, s, "prefix V rows"));
  }
  m->prefix_clean = true;
  return ok();
}

// An entry for the state that ids[0..boundary] ends with: `slot`'s buffers
// (a free or evicted entry), or new ones, with room for its K/V rows after
// the prefix in whole 128-row blocks (decide: state_entry, forward.rs:1048-1080).
int state_entry(dh_model* m, StateEntry* slot, const uint32_t* ids, uint32_t boundary, uint32_t prefix,
                StateEntry& out) {
  const uint32_t rows = boundary - prefix;
  const uint32_t room = (rows + 127) / 128 * 128;
  if (slot) {
    out = std::move(*slot);
    if (out.kv_rows < rows) {
      if (!alloc_kv(m, room, out.k, out.v)) return fail(DH_ENOMEM, "state cache: device allocation failed");
      out.kv_rows = room;
    }
  } else {
    if (!alloc_states(m, out.state, out.conv) || !alloc_kv(m, room, out.k, out.v))
      return fail(DH_ENOMEM, "state cache: device allocation failed");
    out.kv_rows = room;
  }
  out.id = m->next_entry_id++;
  out.ids.assign(ids, ids + boundary);
  return ok();
}

enum class PlanKind { Full, Snapshot, Capture, Hit };
struct Plan {
  PlanKind kind = PlanKind::Full;
  uint32_t boundary = 0;  // Capture
  size_t entry = 0;       // Hit
};

// Run positions start ..= last answer row as `plan` says and read the
// answers' logits into out[index * max_cand + c] (decide: run_answers,
// forward.rs:817-885).
int run_answers(dh_model* m, void* s, const uint32_t* ids, const std::vector<Answer>& answers, Plan plan, float* out) {
  const uint32_t end = answers.back().row + 1;  // tail truncation
  Source src;
  uint32_t start = 0;
  int32_t route = kRouteFull;
  switch (plan.kind) {
    case PlanKind::Full:
      break;
    case PlanKind::Snapshot:
    case PlanKind::Capture:
      src.kind = SourceKind::Snapshot;
      start = (uint32_t)m->snapshot.ids.size();
      route = kRouteSnapshot;
      break;
    case PlanKind::Hit:
      src.kind = SourceKind::State;
      src.entry = plan.entry;
      start = (uint32_t)m->states[plan.entry].ids.size();
      route = kRouteStateCache;
      break;
  }
  m->last_route = route;
  m->last_start = start;
  if (start == 0)
    m->prefix_clean = false;  // this run overwrites the prefix's K/V rows
  else if (!m->prefix_clean)
    TRY(restore_prefix(m, s));
  const uint32_t prefix = m->has_snapshot ? (uint32_t)m->snapshot.ids.size() : 0;
  // a new state's entry: free buffers, or the least recently used entry's
  bool capture = plan.kind == PlanKind::Capture;
  StateEntry entry;
  if (capture) {
    StateEntry slot;
    StateEntry* from = nullptr;
    if (!m->free_entries.empty()) {
      slot = std::move(m->free_entries.back());
      m->free_entries.pop_back();
      from = &slot;
    } else if (m->states.size() >= m->state_capacity) {
      slot = std::move(m->states.back());
      m->states.pop_back();
      if (m->kv_owner == (int64_t)slot.id) m->kv_owner = -1;
      from = &slot;
    }
    TRY(state_entry(m, from, ids, plan.boundary, start, entry));
  }
  // a follow-up needs its entry's K/V rows back unless no run has overwritten them
  const bool restore = plan.kind == PlanKind::Hit && m->kv_owner != (int64_t)m->states[plan.entry].id;

  // stage the span's ids and the answers (decide: stage_embeddings, stage_answers, forward.rs:917-981)
  std::vector<Chunk> chunks = make_chunks(m->chunk, start, end, false, answers);
  if (capture) {
    for (Chunk& ch : chunks)
      if (ch.pos0 < plan.boundary && plan.boundary <= ch.pos0 + ch.rows) ch.capture = plan.boundary - ch.pos0;
  }
  const uint32_t n = (uint32_t)answers.size(), mc = m->cfg.max_cand;
  std::vector<uint32_t> rows(n), pos(n), ncand(n), cand((size_t)n * mc, 0);
  for (const Chunk& ch : chunks)
    for (uint32_t j = ch.a0; j < ch.a0 + ch.n; ++j) rows[j] = answers[j].row - ch.pos0;
  for (uint32_t j = 0; j < n; ++j) {
    pos[j] = answers[j].row;
    ncand[j] = answers[j].ncand;
    std::copy(answers[j].cand, answers[j].cand + answers[j].ncand, cand.begin() + (size_t)j * mc);
  }
  TRY(copy(m->req_ids, ids + start, (uint64_t)(end - start) * 4, hipMemcpyHostToDevice, s, "ids"));
  TRY(copy(m->req_rows, rows.data(), (uint64_t)n * 4, hipMemcpyHostToDevice, s, "answer rows"));
  TRY(copy(m->req_pos, pos.data(), (uint64_t)n * 4, hipMemcpyHostToDevice, s, "answer positions"));
  TRY(copy(m->req_ncand, ncand.data(), (uint64_t)n * 4, hipMemcpyHostToDevice, s, "candidate counts"));
  TRY(copy(m->req_cand, cand.data(), (uint64_t)n * mc * 4, hipMemcpyHostToDevice, s, "candidates"));

  RunArgs r;
  r.ids = m->req_ids;
  r.ans_rows = m->req_rows;
  r.ans_pos = m->req_pos;
  r.cand = m->req_cand;
  r.ncand = m->req_ncand;
  r.logits = m->req_logits;
  int rc = DH_OK;
  if (restore) rc = state_rows(m, s, m->states[plan.entry], prefix, false);
  for (size_t c = 0; c < chunks.size() && rc == DH_OK; ++c) {
    const bool here = capture && chunks[c].capture;
    rc = encode_chunk(m, s, r, chunks[c], src, here ? &entry : nullptr, m->prune);
    // rows prefix..boundary of every K/V cache are final now
    if (rc == DH_OK && here) rc = state_rows(m, s, entry, prefix, true);
  }
  std::vector<float> all((size_t)n * mc);
  if (rc == DH_OK) rc = copy(all.data(), m->req_logits, all.size() * 4, hipMemcpyDeviceToHost, s, "logits");
  if (rc == DH_OK) rc = sync(s);
  // whose K/V rows, from the prefix to the end of its state, the caches now hold
  switch (plan.kind) {
    case PlanKind::Full:
    case PlanKind::Snapshot: m->kv_owner = -1; break;
    case PlanKind::Capture: m->kv_owner = (int64_t)entry.id; break;
    case PlanKind::Hit: m->kv_owner = (int64_t)m->states[plan.entry].id; break;
  }
  if (rc != DH_OK) {
    // the caches' contents and the new entry are unknown
    (void)hipStreamSynchronize(hs(s));
    m->kv_owner = -1;
    if (capture) m->free_entries.push_back(std::move(entry));
    return rc;
  }
  if (plan.kind == PlanKind::Capture) {
    m->states.insert(m->states.begin(), std::move(entry));
  } else if (plan.kind == PlanKind::Hit) {
    StateEntry e = std::move(m->states[plan.entry]);
    m->states.erase(m->states.begin() + (long)plan.entry);
    m->states.insert(m->states.begin(), std::move(e));
  }
  for (uint32_t slot = 0; slot < n; ++slot) {
    const Answer& a = answers[slot];
    const float* row = all.data() + (size_t)slot * mc;
    for (uint32_t c = 0; c < a.ncand; ++c)
      if (!std::isfinite(row[c])) return fail(DH_EDEVICE, "non-finite logits for answer %u (row %u)", a.index, a.row);
    std::copy(row, row + a.ncand, out + (size_t)a.index * mc);
  }
  return ok();
}

}  // namespace

extern "C" {

int dh_state_boundary(const uint32_t* ids, uint32_t len, uint32_t prefix, const uint32_t* marker, uint32_t marker_len,
                      uint32_t limit, uint32_t* boundary, int* found) {
  if (!boundary || !found || (len && !ids) || (marker_len && !marker))
    return fail(DH_EINVAL, "state_boundary: null pointer");
  *boundary = 0;
  *found = state_boundary(ids, len, prefix, marker, marker_len, limit, boundary) ? 1 : 0;
  return ok();
}

int dh_model_set_chunk(dh_model* m, uint32_t rows) {
  if (!m) return fail(DH_EINVAL, "set_chunk: null model");
  if (rows < 1 || rows > m->cfg.max_tokens)
    return fail(DH_EINVAL, "chunk of %u rows; the buffers hold 1 to %u", rows, m->cfg.max_tokens);
  m->chunk = rows;
  return ok();
}

uint32_t dh_model_chunk(const dh_model* m) { return m ? m->chunk : 0; }

void dh_model_set_pruning(dh_model* m, int on) {
  if (m) m->prune = on != 0;
}

int dh_model_pruning(const dh_model* m) { return m && m->prune ? 1 : 0; }

int dh_model_build_snapshot(dh_model* m, void* stream, const uint32_t* prefix_ids, uint32_t len) {
  if (!m) return fail(DH_EINVAL, "build_snapshot: null model");
  TRY(check_ids(m, prefix_ids, len));
  if (len >= m->cfg.max_tokens) return fail(DH_EINVAL, "a %u-token prefix leaves no room for a request", len);
  m->has_snapshot = false;
  m->prefix_clean = false;
  forget_states(m);
  Snapshot snap;
  if (!alloc_states(m, snap.state, snap.conv) || !alloc_kv(m, len, snap.k, snap.v))
    return fail(DH_ENOMEM, "build_snapshot: device allocation failed");
  TRY(copy(m->req_ids, prefix_ids, (uint64_t)len * 4, hipMemcpyHostToDevice, stream, "prefix ids"));
  RunArgs r;
  r.ids = m->req_ids;
  const std::vector<Answer> none;
  for (const Chunk& ch : make_chunks(m->chunk, 0, len, true, none))
    TRY(encode_chunk(m, stream, r, ch, Source{}, nullptr, m->prune));
  for (uint32_t i = 0; i < m->n_lin; ++i) {
    TRY(copy(snap.state[i].as<void>(), m->state[i], kStateBytes, hipMemcpyDeviceToDevice, stream, "snapshot state"));
    TRY(copy(snap.conv[i].as<void>(), m->conv[i], kConvBytes, hipMemcpyDeviceToDevice, stream, "snapshot conv"));
  }
  const uint64_t kv = (uint64_t)len * KV_DIM * 2;
  for (uint32_t a = 0; a < m->n_att; ++a) {
    TRY(copy(snap.k[a].as<void>(), m->kc[a], kv, hipMemcpyDeviceToDevice, stream, "snapshot K rows"));
    TRY(copy(snap.v[a].as<void>(), m->vc[a], kv, hipMemcpyDeviceToDevice, stream, "snapshot V rows"));
  }
  TRY(sync(stream));
  snap.ids.assign(prefix_ids, prefix_ids + len);
  m->snapshot = std::move(snap);
  m->has_snapshot = true;
  m->prefix_clean = true;
  return ok();
}

int dh_model_prefix_len(const dh_model* m, uint32_t* len, int* has_snapshot) {
  if (!m || !len || !has_snapshot) return fail(DH_EINVAL, "prefix_len: null pointer");
  *len = m->has_snapshot ? (uint32_t)m->snapshot.ids.size() : 0;
  *has_snapshot = m->has_snapshot ? 1 : 0;
  return ok();
}

int dh_model_logits(dh_model* m, void* stream, const uint32_t* ids, uint32_t len, const dh_answer* answers,
                    uint32_t n_answers, float* logits, uint32_t flags) {
  if (!m) return fail(DH_EINVAL, "logits: null model");
  if (!logits) return fail(DH_EINVAL, "logits: null output");
  TRY(check_ids(m, ids, len));
  std::vector<Answer> sorted;
  TRY(sorted_answers(m, len, answers, n_answers, sorted));
  Plan plan;
  const uint32_t first_row = sorted.front().row;
  if (!(flags & DH_LOGITS_FULL) && m->has_snapshot && starts_with(ids, len, m->snapshot.ids) &&
      first_row >= m->snapshot.ids.size()) {
    const uint32_t prefix = (uint32_t)m->snapshot.ids.size();
    // a follow-up: the longest cached state the ids start with
    long hit = -1;
    for (size_t i = 0; i < m->states.size(); ++i) {
      const StateEntry& e = m->states[i];
      if (e.ids.size() <= first_row && starts_with(ids, len, e.ids) &&
          (hit < 0 || e.ids.size() > m->states[(size_t)hit].ids.size()))
        hit = (long)i;
    }
    uint32_t boundary = 0;
    if (hit >= 0) {
      plan.kind = PlanKind::Hit;
      plan.entry = (size_t)hit;
    } else if (m->state_capacity > 0 && state_boundary(ids, len, prefix, m->state_marker.data(),
                                                       (uint32_t)m->state_marker.size(), first_row, &boundary)) {
      plan.kind = PlanKind::Capture;
      plan.boundary = boundary;
    } else {
      plan.kind = PlanKind::Snapshot;
    }
  }
  return run_answers(m, stream, ids, sorted, plan, logits);
}

int dh_model_last_route(const dh_model* m, int32_t* route, int64_t* start) {
  if (!m || !route || !start) return fail(DH_EINVAL, "last_route: null pointer");
  *route = m->last_route;
  *start = m->last_start;
  return ok();
}

int dh_model_set_state_cache(dh_model* m, uint32_t entries) {
  if (!m) return fail(DH_EINVAL, "set_state_cache: null model");
  if (entries > kMaxStateEntries)
    return fail(DH_EINVAL, "a state cache of %u entries; at most %u", entries, kMaxStateEntries);
  m->state_capacity = entries;
  if (m->states.size() > entries) m->states.resize(entries);
  const size_t room = entries - m->states.size();
  if (m->free_entries.size() > room) m->free_entries.resize(room);
  bool owner = false;
  for (const StateEntry& e : m->states) owner = owner || (int64_t)e.id == m->kv_owner;
  if (!owner) m->kv_owner = -1;
  return ok();
}

uint32_t dh_model_state_cache_capacity(const dh_model* m) { return m ? m->state_capacity : 0; }

void dh_model_forget_states(dh_model* m) {
  if (m) forget_states(m);
}

uint32_t dh_model_cached_states(const dh_model* m, uint32_t* lens, uint32_t max) {
  if (!m) return 0;
  const uint32_t n = (uint32_t)m->states.size();
  for (uint32_t i = 0; i < n && i < max && lens; ++i) lens[i] = (uint32_t)m->states[i].ids.size();
  return n;
}

int dh_model_set_state_marker(dh_model* m, const uint32_t* marker, uint32_t len) {
  if (!m) return fail(DH_EINVAL, "set_state_marker: null model");
  if (len == 0 || !marker) return fail(DH_EINVAL, "an empty state marker");
  m->state_marker.assign(marker, marker + len);
  forget_states(m);
  return ok();
}

}  // extern "C"
