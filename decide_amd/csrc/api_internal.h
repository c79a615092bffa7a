// Shared by the C-ABI translation units: the context object and the
// status/error helpers (dh_last_error's per-thread message).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "../../include/decide_hip.h"

// One stream's workspaces inside a context. Every stream that makes a split-K
// or forward-kernel call gets its own pair, so calls on different streams that
// share a context can overlap without racing on partials.
struct dh_stream_ws {
  hipStream_t stream = nullptr;
  float* ws = nullptr;   // split-K partials
  uint64_t ws_bytes = 0;
  float* aux = nullptr;  // forward-kernel workspace: the chunked recurrence's per-chunk matrices and attention's
                         // per-piece partial states (never live at the same time)
  uint64_t aux_bytes = 0;
};

struct dh_ctx {
  uint32_t flags = 0;
  int device = 0;
  std::mutex ws_lock;  // guards streams and retired
  std::vector<dh_stream_ws> streams;
  uint64_t ws_cap = 512ull << 20;  // split-K workspace ceiling
  uint32_t cus = 256;              // compute units of the device (sizes attention's key pieces)
  // Workspaces a growth replaced. A captured graph holds the raw pointers it was
  // captured with, so superseded buffers stay allocated until dh_ctx_destroy.
  std::vector<void*> retired;
  float* scratch = nullptr;  // this device's no-allocation scratch (noalloc.hip), kNoAllocScratchBytes
  // dh_gemm_force's plan: variant in the low 32 bits, splits in the high 32; all ones = none
  std::atomic<uint64_t> forced{~0ull};
  std::atomic<uint64_t> used{0};  // bit per distinct kernel launched
};

namespace dh_api {

// Kernel ids for dh_variants_loaded beyond the tile menu (ids < kMaxTileVariants);
// every id is below 64, one bit of dh_ctx::used each.
constexpr int kMaxTileVariants = 24;
enum : int {
  kKidReduce = kMaxTileVariants, kKidReference, kKidGather32, kKidGather16, kKidHead, kKidNorm, kKidFill,
  kKidConv, kKidConvState, kKidDelta, kKidGNorm, kKidQRope, kKidKVRope, kKidAttn, kKidEmbed, kKidFillAny,
  kKidDeltaChunk, kKidStream, kKidAttnCombine, kKidConvDelta, kKidAddNorm, kKidCount
};
static_assert(kKidCount <= 64, "kernel ids must fit dh_ctx::used");

// Records `fmt` as the thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's last error and returns DH_OK.
int ok();
// DH_OK, or DH_ELAUNCH with `what` and HIP's message.
int hip_status(hipError_t e, const char* what);
// Records that kernel `kid` has been launched through this context.
void mark(dh_ctx* c, int kid);
bool aligned(const void* p, uintptr_t a);
// Points *out at `stream`'s forward-kernel workspace, grown to at least `bytes` first if needed (hipMalloc only
// when it grows; the old buffer is retired, not freed). A growth on a stream that is being captured is refused
// with DH_EINVAL: size the workspace with dh_warm_up or an eager call on that stream first.
int ensure_aux(dh_ctx* c, hipStream_t stream, uint64_t bytes, float** out);
// The same for `stream`'s split-K workspace, never beyond c->ws_cap.
int ensure_ws(dh_ctx* c, hipStream_t stream, uint64_t bytes, float** out);
// dh_gemm_force's plan, if one is set: true with the variant and splits.
bool forced_plan(const dh_ctx* c, int* variant, uint32_t* splits);
// dh_attention with a bound on the rows' positions (every qpos[r] < npos), which sizes the key pieces; the
// forward knows it (the chunk's last position + 1).
int attention_run(dh_ctx* ctx, void* stream, const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                  const float* pq, const uint32_t* qpos, uint16_t* y, uint32_t rows, uint32_t ldq, uint32_t npos);

}  // namespace dh_api
