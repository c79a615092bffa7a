// The C ABI (include/decide_hip.h): contract checks, planning, launches.
//
// Contract checks restate decide's Gemm::gemm asserts
// (crates/decide-engine/src/kernels/gemm.rs:140-163) and Norm::rmsnorm's
// (kernels/norm.rs:27), returning DH_EINVAL with the same wording instead of
// panicking; nothing is launched after a failed check.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/decide_hip.h"
#include "api_internal.h"
#include "dh_kernels.h"
#include "plan.h"

namespace dh_api {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return DH_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(DH_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
}

void mark(dh_ctx* c, int kid) {
  if (kid >= 0 && kid < 64) c->used.fetch_or(1ull << kid, std::memory_order_relaxed);
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

bool forced_plan(const dh_ctx* c, int* variant, uint32_t* splits) {
  const uint64_t f = c ? c->forced.load(std::memory_order_relaxed) : ~0ull;
  if (f == ~0ull) return false;
  *variant = (int)(uint32_t)f;
  *splits = (uint32_t)(f >> 32);
  return true;
}

namespace {
// Grows one of `stream`'s workspaces (`aux` selects which) to at least `bytes`:
// by at least half its size, so a run of small growths retires little, or
// exactly `bytes` when the larger request fails. The old buffer joins
// c->retired.
int grow(dh_ctx* c, hipStream_t stream, bool aux, uint64_t bytes, uint64_t cap, const char* what, float** out) {
  std::lock_guard<std::mutex> g(c->ws_lock);
  dh_stream_ws* sw = nullptr;
  for (dh_stream_ws& e : c->streams)
    if (e.stream == stream) sw = &e;
  if (!sw) {
    c->streams.push_back(dh_stream_ws{});
    sw = &c->streams.back();
    sw->stream = stream;
  }
  float** buf = aux ? &sw->aux : &sw->ws;
  uint64_t* have = aux ? &sw->aux_bytes : &sw->ws_bytes;
  if (bytes <= *have) {
    *out = *buf;
    return DH_OK;
  }
  if (bytes > cap)
    return fail(DH_ENOMEM, "%s of %llu bytes exceeds its %llu-byte ceiling", what, (unsigned long long)bytes,
                (unsigned long long)cap);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(DH_EINVAL,
                "%s must grow to %llu bytes on a stream that is being captured; size it first with dh_warm_up "
                "or an eager call of the same size on this stream",
                what, (unsigned long long)bytes);
  uint64_t want = std::min(cap, std::max(bytes, *have + *have / 2));
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess && want > bytes) {
    (void)hipGetLastError();
    want = bytes;
    e = hipMalloc(&p, want);
  }
  if (e != hipSuccess)
    return fail(DH_ENOMEM, "%s of %llu bytes: %s", what, (unsigned long long)want, hipGetErrorString(e));
  if (*buf) c->retired.push_back(*buf);
  *buf = (float*)p;
  *have = want;
  *out = *buf;
  return DH_OK;
}
}  // namespace

int ensure_aux(dh_ctx* c, hipStream_t stream, uint64_t bytes, float** out) {
  return grow(c, stream, true, bytes, UINT64_MAX, "forward workspace", out);
}

int ensure_ws(dh_ctx* c, hipStream_t stream, uint64_t bytes, float** out) {
  return grow(c, stream, false, bytes, c->ws_cap, "split-K workspace", out);
}

}  // namespace dh_api

using namespace dh_api;

namespace {

// gemm.rs:140-144: what every implementation asserts.
int check_gemm_common(const void* x, uint32_t ldx, const void* w, uint32_t ldw, const void* y, uint32_t ldy,
                      uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  if (epi > 3u) return fail(DH_EINVAL, "gemm: epilogue %u is not one of 0..3", epi);
  if (n % 32 != 0 || k % 32 != 0)
    return fail(DH_EINVAL, "gemm: N = %u and K = %u must be multiples of 32", n, k);
  if (m < 1) return fail(DH_EINVAL, "gemm: M must be at least 1");
  if (ldx < k || ldw < k)
    return fail(DH_EINVAL, "gemm: row strides ldx = %u, ldw = %u must cover K = %u", ldx, ldw, k);
  const uint32_t y_cols = epi == DH_EPI_SWIGLU_F16 ? n / 2 : n;
  if (ldy < y_cols) return fail(DH_EINVAL, "gemm: row stride ldy = %u must cover the %u output columns", ldy, y_cols);
  if (!x || !w || !y) return fail(DH_EINVAL, "gemm: null operand");
  return DH_OK;
}

// gemm.rs:159-163: the fast kernels' extra requirements (decide's baseline
// returns before these asserts, gemm.rs:150-156), plus this build's 4 GiB
// row-span limit of the tile kernel's DMA offsets.
int check_gemm_fast(const void* x, uint32_t ldx, const void* w, uint32_t ldw, const void* y, uint32_t ldy,
                    uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  if (ldx % 8 != 0 || ldw % 8 != 0)
    return fail(DH_EINVAL, "gemm (fast): ldx = %u and ldw = %u must be multiples of 8", ldx, ldw);
  if (!aligned(x, 16) || !aligned(w, 16))
    return fail(DH_EINVAL, "gemm (fast): x/w addresses %p/%p must be multiples of 16", x, w);
  if (ldy % 2 != 0) return fail(DH_EINVAL, "gemm (fast): ldy = %u must be even", ldy);
  const uintptr_t y_align = (epi == DH_EPI_STORE_F32 || epi == DH_EPI_ADD_F32) ? 8 : 4;
  if (!aligned(y, y_align)) return fail(DH_EINVAL, "gemm (fast): y address %p must be a multiple of %u", y, (unsigned)y_align);
  // The tile kernel's DMA addresses a row as a 32-bit byte offset from the operand's base.
  if ((uint64_t)(m - 1) * ldx * 2 + (uint64_t)k * 2 > UINT32_MAX)
    return fail(DH_EINVAL, "gemm: X rows span more than 4 GiB (m = %u, ldx = %u); split the call along M", m, ldx);
  if ((uint64_t)(n ? n - 1 : 0) * ldw * 2 + (uint64_t)k * 2 > UINT32_MAX)
    return fail(DH_EINVAL, "gemm: W rows span more than 4 GiB (n = %u, ldw = %u); split the call along N", n, ldw);
  return DH_OK;
}

// The reference kernel reads and writes single elements: only their natural alignment is needed.
int check_gemm_reference(const void* x, const void* w, const void* y, uint32_t epi) {
  const uintptr_t y_align = (epi == DH_EPI_STORE_F32 || epi == DH_EPI_ADD_F32) ? 4 : 2;
  if (!aligned(x, 2) || !aligned(w, 2) || !aligned(y, y_align))
    return fail(DH_EINVAL, "gemm (reference): x/w/y addresses %p/%p/%p must be aligned to their element sizes", x,
                w, y);
  return DH_OK;
}

int check_gemm(const dh_ctx* c, const void* x, uint32_t ldx, const void* w, uint32_t ldw, const void* y,
               uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  int rc = check_gemm_common(x, ldx, w, ldw, y, ldy, m, n, k, epi);
  if (rc != DH_OK) return rc;
  if (c && (c->flags & DH_GEMM_REFERENCE)) return check_gemm_reference(x, w, y, epi);
  return check_gemm_fast(x, ldx, w, ldw, y, ldy, m, n, k, epi);
}

dh::Plan choose_plan(const dh_ctx* c, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  int fv;
  uint32_t fs;
  if (forced_plan(c, &fv, &fs)) return dh::plan_make(fv, std::max(1u, fs), m, n, k, epi);
  return dh::plan_gemm(m, n, k, epi, c ? c->ws_cap : (512ull << 20));
}

// Enqueues plan p. Split-K partials go to `fixed_ws` when given (it must hold
// p.ws_bytes), else to the context's workspace, grown if needed. With
// `partials_out`, a split plan stops after the tile kernel and returns where
// its partials are, for the caller to reduce.
int launch_plan(dh_ctx* c, hipStream_t s, const dh::Plan& p, const void* x, uint32_t ldx, uint32_t m, uint32_t k,
                const dh_gemm_member* mem, uint32_t count, float* fixed_ws = nullptr,
                const float** partials_out = nullptr) {
  dh::TileArgs a{};
  a.x = (const _Float16*)x;
  a.ldx = ldx;
  a.m = m;
  a.k = k;
  a.mtiles = p.mtiles;
  a.splits = p.splits;
  a.kps = p.kps;
  a.count = count;
  const bool stream = p.variant == dh::kStreamVariant;
  const uint32_t bn = stream ? 32u : (uint32_t)dh::variant_info(p.variant).bn();
  uint32_t stripes = 0;
  for (uint32_t i = 0; i < count; ++i) {
    a.mem[i].w = (const _Float16*)mem[i].w;
    a.mem[i].y = mem[i].y;
    a.mem[i].ldw = mem[i].ldw;
    a.mem[i].ldy = mem[i].ldy;
    a.mem[i].n = mem[i].n;
    a.mem[i].epi = mem[i].epi;
    a.mem[i].stripe_begin = stripes;
    stripes += (mem[i].n + bn - 1) / bn;
  }
  a.nstripes = stripes;
  if (stripes == 0) return ok();  // N = 0: nothing to compute
  const uint64_t grid64 = (uint64_t)p.mtiles * stripes * p.splits;
  if (grid64 > (uint64_t)INT32_MAX)
    return fail(DH_EINVAL, "gemm: %llu workgroups exceed one launch; split the call along M or N",
                (unsigned long long)grid64);
  const uint32_t grid = (uint32_t)grid64;
  if (!stream) {
    dh::Plan po = p;
    po.stripes = stripes;  // a grouped launch counts each member's own stripes
    po.grid = grid;
    a.ngroup = dh::plan_order(po);
  }
  if (p.splits > 1) {
    if (count != 1) return fail(DH_EINVAL, "gemm: split-K needs a single member");
    if (fixed_ws) {
      a.ws = fixed_ws;
    } else {
      int rc = ensure_ws(c, s, p.ws_bytes, &a.ws);
      if (rc != DH_OK) return rc;
    }
  }
  int rc;
  if (stream) {
    mark(c, kKidStream);
    rc = hip_status(dh::launch_stream(a, grid, s), "gemm streaming kernel launch");
  } else {
    mark(c, p.variant);
    rc = hip_status(dh::launch_tile(p.variant, a, grid, s), "gemm tile kernel launch");
  }
  if (rc != DH_OK || p.splits == 1) return rc;
  if (partials_out) {
    *partials_out = a.ws;
    return rc;
  }
  mark(c, kKidReduce);
  return hip_status(dh::launch_splitk_reduce(a.ws, p.splits, m, mem[0].n, mem[0].y, mem[0].ldy, mem[0].epi, s),
                    "split-K reduce launch");
}

}  // namespace

extern "C" {

const char* dh_last_error(void) { return g_err.c_str(); }

const char* dh_version(void) { return "decide-hip 0.1.0 (gfx950, fp16 MFMA 16x16x32)"; }

int dh_ctx_create(uint32_t flags, dh_ctx** out) {
  if (!out) return fail(DH_EINVAL, "dh_ctx_create: out is NULL");
  *out = nullptr;
  if ((flags & DH_DELTA_CHUNKED) && (flags & DH_DELTA_SEQUENTIAL))
    return fail(DH_EINVAL, "ctx_create: DH_DELTA_CHUNKED and DH_DELTA_SEQUENTIAL exclude each other");
  if (flags & ~(DH_GEMM_REFERENCE | DH_DELTA_CHUNKED | DH_DELTA_SEQUENTIAL))
    return fail(DH_EINVAL, "dh_ctx_create: unknown flags 0x%x", flags);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DH_EDEVICE, "dh_ctx_create: no HIP device: %s", hipGetErrorString(e));
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return fail(DH_EDEVICE, "dh_ctx_create: hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(DH_EDEVICE, "dh_ctx_create: device %d is %s; this library is built for gfx950", dev, prop.gcnArchName);
  float* scratch = nullptr;
  e = dh::noalloc_scratch(dev, &scratch);
  if (e != hipSuccess)
    return fail(DH_EDEVICE, "dh_ctx_create: no-allocation scratch of device %d: %s", dev, hipGetErrorString(e));
  dh_ctx* c = new dh_ctx();
  c->flags = flags;
  c->device = dev;
  c->scratch = scratch;
  c->cus = prop.multiProcessorCount > 0 ? (uint32_t)prop.multiProcessorCount : 256u;
  *out = c;
  return ok();
}

void dh_ctx_destroy(dh_ctx* ctx) {
  if (!ctx) return;
  for (const dh_stream_ws& e : ctx->streams) {
    if (e.ws) (void)hipFree(e.ws);
    if (e.aux) (void)hipFree(e.aux);
  }
  for (void* p : ctx->retired) (void)hipFree(p);
  delete ctx;
}

uint32_t dh_variants_loaded(const dh_ctx* ctx) {
  return ctx ? (uint32_t)__builtin_popcountll(ctx->used.load(std::memory_order_relaxed)) : 0u;
}

int dh_gemm_nt(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y,
               uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  int rc = check_gemm(ctx, x, ldx, w, ldw, y, ldy, m, n, k, epi);
  if (rc != DH_OK) return rc;
  if (!ctx) return fail(DH_EINVAL, "gemm: null context");
  hipStream_t s = (hipStream_t)stream;
  if (ctx->flags & DH_GEMM_REFERENCE) {
    mark(ctx, kKidReference);
    return hip_status(dh::launch_gemm_reference((const _Float16*)x, ldx, (const _Float16*)w, ldw, y, ldy, m, n, k,
                                                epi, s),
                      "gemm reference kernel launch");
  }
  const dh::Plan p = choose_plan(ctx, m, n, k, epi);
  if (p.variant < 0) return fail(DH_EINVAL, "gemm: no plan for M = %u, N = %u, K = %u", m, n, k);
  dh_gemm_member mem{w, y, ldw, ldy, n, epi};
  return launch_plan(ctx, s, p, x, ldx, m, k, &mem, 1);
}

int dh_gemm_add_rmsnorm(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, float* y,
                        uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, const float* norm_w, uint32_t add_one,
                        float eps, uint16_t* h, uint32_t ldh) {
  int rc = check_gemm(ctx, x, ldx, w, ldw, y, ldy, m, n, k, DH_EPI_ADD_F32);
  if (rc != DH_OK) return rc;
  if (!ctx) return fail(DH_EINVAL, "gemm_add_rmsnorm: null context");
  if (n == 0) return fail(DH_EINVAL, "gemm_add_rmsnorm: N must be at least 32 (a row to normalise)");
  if (n > ldh) return fail(DH_EINVAL, "gemm_add_rmsnorm: N = %u exceeds ldh = %u", n, ldh);
  if (m && (!norm_w || !h)) return fail(DH_EINVAL, "gemm_add_rmsnorm: null norm weight or output");
  hipStream_t s = (hipStream_t)stream;
  if (!(ctx->flags & DH_GEMM_REFERENCE) && m && k) {
    const dh::Plan p = choose_plan(ctx, m, n, k, DH_EPI_ADD_F32);
    if (p.variant >= 0 && p.splits > 1 && dh::splitk_add_rmsnorm_fits(p.splits, n, ldy, ldh, y, norm_w, h)) {
      dh_gemm_member mem{w, y, ldw, ldy, n, DH_EPI_ADD_F32};
      const float* partials = nullptr;
      rc = launch_plan(ctx, s, p, x, ldx, m, k, &mem, 1, nullptr, &partials);
      if (rc != DH_OK) return rc;
      mark(ctx, kKidAddNorm);
      return hip_status(dh::launch_splitk_add_rmsnorm(partials, p.splits, m, n, y, ldy, norm_w, (_Float16*)h, ldh,
                                                      add_one != 0, eps, s),
                        "split-K add + rmsnorm launch");
    }
  }
  rc = dh_gemm_nt(ctx, stream, x, ldx, w, ldw, y, ldy, m, n, k, DH_EPI_ADD_F32);
  if (rc != DH_OK) return rc;
  mark(ctx, kKidNorm);
  return hip_status(dh::launch_rmsnorm_rows(y, norm_w, (_Float16*)h, nullptr, m, n, ldy, ldh, add_one != 0, eps, s),
                    "rmsnorm_rows");
}

static_assert(dh::kNoAllocScratchBytes == DH_NOALLOC_SCRATCH_BYTES, "the header states the scratch size");

int dh_gemm_nt_noalloc(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, const void* w, uint32_t ldw, void* y,
                       uint32_t ldy, uint32_t m, uint32_t n, uint32_t k, uint32_t epi) {
  int rc = check_gemm(ctx, x, ldx, w, ldw, y, ldy, m, n, k, epi);
  if (rc != DH_OK) return rc;
  if (!ctx) return fail(DH_EINVAL, "gemm (no-alloc): null context");
  if (!ctx->scratch) return fail(DH_EDEVICE, "gemm (no-alloc): the context has no device scratch");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != ctx->device)
    return fail(DH_EINVAL, "gemm (no-alloc): the context belongs to device %d, device %d is current", ctx->device,
                dev);
  hipStream_t s = (hipStream_t)stream;
  if (ctx->flags & DH_GEMM_REFERENCE) {
    mark(ctx, kKidReference);
    return hip_status(dh::launch_gemm_reference((const _Float16*)x, ldx, (const _Float16*)w, ldw, y, ldy, m, n, k,
                                                epi, s),
                      "gemm reference kernel launch");
  }
  int fv;
  uint32_t fs;
  const dh::Plan p = forced_plan(ctx, &fv, &fs) ? dh::plan_make(fv, std::max(1u, fs), m, n, k, epi)
                                                : dh::plan_gemm(m, n, k, epi, dh::kNoAllocScratchBytes);
  if (p.variant < 0) return fail(DH_EINVAL, "gemm (no-alloc): no plan for M = %u, N = %u, K = %u", m, n, k);
  if (p.ws_bytes > dh::kNoAllocScratchBytes)
    return fail(DH_EINVAL,
                "gemm (no-alloc): M = %u, N = %u with %u K splits needs %llu bytes of scratch; this entry point "
                "holds %llu",
                m, n, p.splits, (unsigned long long)p.ws_bytes, (unsigned long long)dh::kNoAllocScratchBytes);
  dh_gemm_member mem{w, y, ldw, ldy, n, epi};
  return launch_plan(ctx, s, p, x, ldx, m, k, &mem, 1, ctx->scratch);
}

int dh_gemm_nt_grouped(dh_ctx* ctx, void* stream, const void* x, uint32_t ldx, uint32_t m, uint32_t k,
                       const dh_gemm_member* members, uint32_t count) {
  if (!members || count < 1 || count > (uint32_t)dh::kMaxMembers)
    return fail(DH_EINVAL, "gemm grouped: count = %u must be in 1..%d", count, dh::kMaxMembers);
  uint32_t n_total = 0;
  uint32_t ns[dh::kMaxMembers];
  for (uint32_t i = 0; i < count; ++i) {
    const dh_gemm_member& mb = members[i];
    ns[i] = mb.n;
    int rc = check_gemm(ctx, x, ldx, mb.w, mb.ldw, mb.y, mb.ldy, m, mb.n, k, mb.epi);
    if (rc != DH_OK) {
      std::string msg = g_err;
      return fail(rc, "member %u: %s", i, msg.c_str());
    }
    n_total += mb.n;
  }
  if (!ctx) return fail(DH_EINVAL, "gemm grouped: null context");
  hipStream_t s = (hipStream_t)stream;
  if (ctx->flags & DH_GEMM_REFERENCE) {
    mark(ctx, kKidReference);
    for (uint32_t i = 0; i < count; ++i) {
      const dh_gemm_member& mb = members[i];
      int rc = hip_status(dh::launch_gemm_reference((const _Float16*)x, ldx, (const _Float16*)mb.w, mb.ldw, mb.y,
                                                    mb.ldy, m, mb.n, k, mb.epi, s),
                          "gemm reference kernel launch");
      if (rc != DH_OK) return rc;
    }
    return ok();
  }
  int fv;
  uint32_t fs;
  dh::Plan p = forced_plan(ctx, &fv, &fs) ? dh::plan_make(fv, 1, m, n_total, k, 0u) : dh::plan_grouped(m, k, ns, count);
  if (p.variant < 0) return fail(DH_EINVAL, "gemm grouped: no plan");
  return launch_plan(ctx, s, p, x, ldx, m, k, members, count);
}

static_assert(dh::kStreamVariant == (int)DH_GEMM_STREAM_VARIANT, "the streaming kernel's plan id");

int dh_gemm_plan_for(const dh_ctx* ctx, uint32_t m, uint32_t n, uint32_t k, uint32_t epi, dh_gemm_plan* out) {
  if (!out) return fail(DH_EINVAL, "dh_gemm_plan_for: out is NULL");
  if (epi > 3u || m < 1 || n % 32 || k % 32) return fail(DH_EINVAL, "dh_gemm_plan_for: invalid shape");
  const dh::Plan p = choose_plan(ctx, m, n, k, epi);
  if (p.variant < 0) return fail(DH_EINVAL, "dh_gemm_plan_for: no plan");
  out->variant = (uint32_t)p.variant;
  if (p.variant == dh::kStreamVariant) {
    out->bm = dh::kStreamMaxM;
    out->bn = 32;
    out->waves = 4;
  } else {
    const dh::VariantInfo vi = dh::variant_info(p.variant);
    out->bm = (uint32_t)vi.bm();
    out->bn = (uint32_t)vi.bn();
    out->waves = (uint32_t)vi.waves();
  }
  out->splits = p.splits;
  out->workgroups = p.grid;
  out->ws_bytes = p.ws_bytes;
  out->order = dh::plan_order(p);
  return ok();
}

int dh_gemm_ws_need(const dh_ctx* ctx, uint32_t max_m, uint32_t n, uint32_t k, uint64_t* out) {
  if (!out) return fail(DH_EINVAL, "dh_gemm_ws_need: out is NULL");
  if (max_m < 1 || n % 32 || k % 32) return fail(DH_EINVAL, "dh_gemm_ws_need: invalid shape");
  if (max_m > DH_PLAN_MAX_ROWS)
    return fail(DH_EINVAL, "dh_gemm_ws_need: max_m = %u exceeds %u (DH_PLAN_MAX_ROWS)", max_m, DH_PLAN_MAX_ROWS);
  *out = dh::plan_ws_need(max_m, n, k, ctx ? ctx->ws_cap : (512ull << 20));
  return ok();
}

int dh_gemm_force(dh_ctx* ctx, uint32_t variant, uint32_t splits) {
  if (!ctx) return fail(DH_EINVAL, "dh_gemm_force: null context");
  if (variant == UINT32_MAX) {
    ctx->forced.store(~0ull, std::memory_order_relaxed);
    return ok();
  }
  if (variant >= (uint32_t)dh::variant_count())
    return fail(DH_EINVAL, "dh_gemm_force: variant %u >= %d", variant, dh::variant_count());
  if (splits < 1 || splits > 64) return fail(DH_EINVAL, "dh_gemm_force: splits = %u must be in 1..64", splits);
  ctx->forced.store((uint64_t)splits << 32 | variant, std::memory_order_relaxed);
  return ok();
}

uint32_t dh_gemm_variant_count(void) { return (uint32_t)dh::variant_count(); }

int dh_gemm_variant_info(uint32_t variant, uint32_t* bm, uint32_t* bn, uint32_t* waves, uint32_t* wave_cols) {
  if (variant >= (uint32_t)dh::variant_count()) return fail(DH_EINVAL, "variant %u out of range", variant);
  const dh::VariantInfo vi = dh::variant_info((int)variant);
  if (bm) *bm = (uint32_t)vi.bm();
  if (bn) *bn = (uint32_t)vi.bn();
  if (waves) *waves = (uint32_t)vi.waves();
  if (wave_cols) *wave_cols = (uint32_t)(16 * vi.fn);
  return ok();
}

int dh_warm_up(dh_ctx* ctx, void* stream, uint32_t max_m) {
  if (!ctx) return fail(DH_EINVAL, "dh_warm_up: null context");
  if (max_m > DH_PLAN_MAX_ROWS)
    return fail(DH_EINVAL, "dh_warm_up: max_m = %u exceeds %u (DH_PLAN_MAX_ROWS)", max_m, DH_PLAN_MAX_ROWS);
  hipStream_t s = (hipStream_t)stream;
  // Size the workspace for the largest split-K plan of decide's engine shapes
  // (gemm_configs.rs:385) at any M up to max_m rows, so no such call grows it.
  static const uint32_t kShapes[][2] = {{2560, 12352}, {2560, 10240}, {2560, 18432}, {4096, 2560},
                                        {9216, 2560},  {2560, 2048},  {2560, 8192},  {2560, 6144}};
  uint64_t need = 0;
  int fv;
  uint32_t fs;
  if (!forced_plan(ctx, &fv, &fs) && !(ctx->flags & DH_GEMM_REFERENCE))
    for (auto& kn : kShapes) need = std::max(need, dh::plan_ws_need(std::max(1u, max_m), kn[1], kn[0], ctx->ws_cap));
  float* unused = nullptr;
  if (need) {
    int rc = ensure_ws(ctx, s, need, &unused);
    if (rc != DH_OK) return rc;
  }
  const bool chunked = (ctx->flags & DH_DELTA_CHUNKED) ||
                       (!(ctx->flags & DH_DELTA_SEQUENTIAL) && max_m >= DH_DELTA_CHUNK_MIN_T);
  // the forward-kernel workspace: the chunked recurrence's for max_m tokens, attention's key pieces for max_m rows
  uint64_t aux = dh::attention_ws_max(max_m);
  if (chunked) aux = std::max<uint64_t>(aux, dh::delta_chunk_ws_floats(std::max(1u, max_m)) * sizeof(float));
  if (aux) {
    int rc = ensure_aux(ctx, s, aux, &unused);
    if (rc != DH_OK) return rc;
  }
  // One tiny launch of every tile variant (M = 16, N = bn, K = 64) and of the
  // streaming kernel (M = 16, N = 32, K = 128) into scratch.
  void* scratch = nullptr;
  const size_t xb = 16 * 128 * 2, wb = 512 * 64 * 2, yb = 16 * 512 * 4;
  hipError_t e = hipMalloc(&scratch, xb + wb + yb);
  if (e != hipSuccess) return fail(DH_ENOMEM, "dh_warm_up: %s", hipGetErrorString(e));
  e = hipMemsetAsync(scratch, 0, xb + wb + yb, s);
  int rc = hip_status(e, "dh_warm_up memset");
  char* base = (char*)scratch;
  for (int v = 0; v < dh::variant_count() && rc == DH_OK; ++v) {
    const dh::VariantInfo vi = dh::variant_info(v);
    dh_gemm_member mem{base + xb, base + xb + wb, 64, (uint32_t)vi.bn(), (uint32_t)vi.bn(), DH_EPI_STORE_F32};
    rc = launch_plan(ctx, s, dh::plan_make(v, 1, 16, vi.bn(), 64, 0u), base, 64, 16, 64, &mem, 1);
  }
  if (rc == DH_OK) {
    dh_gemm_member mem{base + xb, base + xb + wb, 128, 32, 32, DH_EPI_STORE_F32};
    rc = launch_plan(ctx, s, dh::plan_stream(16, 32, 128, 0), base, 128, 16, 128, &mem, 1);
  }
  if (rc == DH_OK && need) {
    // and the split-K reduction once (two splits of K = 128)
    const dh::VariantInfo vi = dh::variant_info(0);
    dh_gemm_member mem{base + xb, base + xb + wb, 128, (uint32_t)vi.bn(), (uint32_t)vi.bn(), DH_EPI_STORE_F32};
    rc = launch_plan(ctx, s, dh::plan_make(0, 2, 8, vi.bn(), 128, 0u), base, 128, 8, 128, &mem, 1);
  }
  if (rc == DH_OK) {
    e = hipStreamSynchronize(s);
    rc = hip_status(e, "dh_warm_up sync");
  }
  (void)hipFree(scratch);
  return rc == DH_OK ? ok() : rc;
}

int dh_gather_rows_f32(dh_ctx* ctx, void* stream, const float* x, const uint32_t* rowmap, float* out, uint32_t rows,
                       uint32_t h) {
  if (!ctx) return fail(DH_EINVAL, "gather_rows_f32: null context");
  if (rows && (!x || !rowmap || !out)) return fail(DH_EINVAL, "gather_rows_f32: null pointer");
  mark(ctx, kKidGather32);
  return hip_status(dh::launch_gather_rows(x, rowmap, out, rows, h, 4, (hipStream_t)stream), "gather_rows_f32");
}

int dh_gather_rows_f16(dh_ctx* ctx, void* stream, const uint16_t* x, const uint32_t* rowmap, uint16_t* out,
                       uint32_t rows, uint32_t h) {
  if (!ctx) return fail(DH_EINVAL, "gather_rows_f16: null context");
  if (rows && (!x || !rowmap || !out)) return fail(DH_EINVAL, "gather_rows_f16: null pointer");
  mark(ctx, kKidGather16);
  return hip_status(dh::launch_gather_rows(x, rowmap, out, rows, h, 2, (hipStream_t)stream), "gather_rows_f16");
}

int dh_final_head(dh_ctx* ctx, void* stream, const float* x, const float* w, const uint16_t* table,
                  const uint32_t* cand, const uint32_t* ncand, float* logits, uint32_t rows, uint32_t hidden,
                  uint32_t max_cand, float eps) {
  if (hidden == 0 || hidden % 8 != 0 || hidden > 16384)
    return fail(DH_EINVAL, "final_head: hidden = %u must be a positive multiple of 8, at most 16384", hidden);
  if (max_cand < 1 || max_cand > 524280u)
    return fail(DH_EINVAL, "final_head: max_cand = %u must be in 1..524280", max_cand);
  if (!aligned(table, 16)) return fail(DH_EINVAL, "final_head: table address %p must be a multiple of 16", table);
  if (!(eps > 0.0f)) return fail(DH_EINVAL, "final_head: eps must be positive");
  if (!ctx) return fail(DH_EINVAL, "final_head: null context");
  if (rows && (!x || !w || !table || !cand || !ncand || !logits)) return fail(DH_EINVAL, "final_head: null pointer");
  mark(ctx, kKidHead);
  return hip_status(dh::launch_final_head(x, w, table, cand, ncand, logits, rows, hidden, max_cand, eps,
                                          (hipStream_t)stream),
                    "final_head");
}

int dh_rmsnorm_rows(dh_ctx* ctx, void* stream, const float* x, const float* w, uint16_t* y, const uint32_t* rowmap,
                    uint32_t rows, uint32_t h, uint32_t ld_in, uint32_t ld_out, uint32_t add_one, float eps) {
  if (h > ld_in || h > ld_out)
    return fail(DH_EINVAL, "rmsnorm: H = %u exceeds a row stride (ld_in = %u, ld_out = %u)", h, ld_in, ld_out);
  if (h == 0) return fail(DH_EINVAL, "rmsnorm: H must be at least 1");
  if (!ctx) return fail(DH_EINVAL, "rmsnorm: null context");
  if (rows && (!x || !w || !y || !rowmap)) return fail(DH_EINVAL, "rmsnorm: null pointer");
  mark(ctx, kKidNorm);
  return hip_status(dh::launch_rmsnorm_rows(x, w, (_Float16*)y, rowmap, rows, h, ld_in, ld_out, add_one != 0, eps,
                                            (hipStream_t)stream),
                    "rmsnorm_rows");
}

int dh_fill_normal_f16(dh_ctx* ctx, void* stream, uint16_t* out, uint64_t n, uint64_t seed, float std) {
  if (!ctx) return fail(DH_EINVAL, "fill_normal_f16: null context");
  if (n && !out) return fail(DH_EINVAL, "fill_normal_f16: null pointer");
  if (!(std >= 0.0f) || !std::isfinite(std)) return fail(DH_EINVAL, "fill_normal_f16: std must be finite and >= 0");
  mark(ctx, kKidFill);
  return hip_status(dh::launch_fill_normal_f16(out, n, seed, std, (hipStream_t)stream), "fill_normal_f16");
}

}  // extern "C"
