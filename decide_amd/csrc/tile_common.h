// Device helpers of the MFMA tile GEMM kernels (gemm_tile.hip):
// vector types, compile-time loops, the SwiGLU value, the XCD renumbering and
// the inline-asm hot-loop blocks (LDS reads, MFMA, waits, DMA). Device code
// only; include from HIP sources.
#pragma once

#include <type_traits>

#include "dh_kernels.h"

namespace dh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename Fn>
__device__ __forceinline__ void static_for(Fn&& fn) {
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    static_for<B + 1, E>(fn);
  }
}

// silu(v) = v / (1 + e^-v) with the hardware exp and reciprocal (about 1 ulp
// each); decide's kernels use fast-math exp for silu as well (common.h:5-7).
__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// SwiGLU value silu(g) · u in fp32 (one helper for every epilogue, so all
// kernels and tilings evaluate it with the same instructions). The product
// is materialised in fp32 (decide rounds it to fp32, then to half): left
// alone, the compiler may fuse the multiply with the fp16 conversion that
// follows into one v_fma_mix, which rounds once and so stores other bits.
__device__ __forceinline__ float swiglu_f(float g, float u) {
  float v = silu_f(g) * u;
  asm("" : "+v"(v));
  return v;
}

// Keeps an accumulator fragment in AGPRs up to this point of the epilogue, so
// that the fragments move to VGPRs one at a time as they are stored; left to
// itself the compiler copies them all at the loop exit, which for the largest
// tiles needs more VGPRs than there are.
__device__ __forceinline__ void pin_acc(f4& v) { asm volatile("" : "+a"(v)); }

// Workgroup b runs on XCD b % 8. Renumber so XCD x owns one contiguous range
// of work ids (a bijection on [0, G)).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t G) {
  const uint32_t xcd = b & 7u, local = b >> 3;
  const uint32_t per = G >> 3, rem = G & 7u;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// ---------------------------------------------------------------------------
// Hot-loop building blocks, written as inline asm so they issue exactly in
// program order and the accumulators stay pinned in AGPRs.
// LDS 16-byte read at LDS byte address base + OFF (OFF < 65536).
template <int OFF>
__device__ __forceinline__ void ds_read16(h8& dst, uint32_t base) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "n"(OFF));
}

template <int N>
__device__ __forceinline__ void wait_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}

// MFMA as volatile asm: stays in program order with the reads and waits.
__device__ __forceinline__ void mfma_acc_v(f4& acc, const h8& a, const h8& b) {
  asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void tie(h8& v) { asm volatile("" : "+v"(v)); }

// 16-byte-per-lane DMA global → LDS: lane l's 16 bytes at sbase + voff land at
// LDS byte address m0 + 16·l. M0 is written in the same statement; one wait
// state separates the write from its use.
// M0 is a reserved register to the compiler, which warns that it may not be
// preserved across the statement; nothing else in these kernels reads M0
// (the build checks the generated code for other M0 uses).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(uint32_t m0, uint32_t voff, const void* sbase) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:0" ::"s"(m0), "v"(voff), "s"(sbase)
               : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace dh
