// Measurement probe (not part of the library): how fast one CU can pull data
// from L2 (or HBM) into LDS with global_load_lds_dwordx4, the DMA every GEMM
// tile stage is fed by, as a function of the waves issuing it, with plain
// global_load_dwordx4 into registers beside it; then how fast the CU's waves
// read LDS back with ds_read_b128 (the MFMA operand reads), alone and with
// DMA writes landing in LDS at the same time. One workgroup per CU; each
// wave issues `depth` 1 KB loads, waits for them, and repeats over its own
// window of a buffer that either fits L2 (2 MB, re-read) or does not (1 GB,
// streamed from HBM). Both sizes are powers of two, so addresses wrap with a
// mask: a 64-bit `%` here would compile to a software division per load and
// measure that instead of the memory system. The DMA's base comes from
// readfirstlane, so the asm statement supplies the 5 wait states a VMEM read
// of a VALU-written SGPR needs (s_mov + s_nop 4).
//
// Build and run: make -C decide_amd/csrc probe && decide_amd/csrc/_build/l2_probe
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#pragma clang diagnostic ignored "-Winline-asm"

typedef float f4 __attribute__((ext_vector_type(4)));

// byte offset of load n of iteration `it` for `wave`, wrapped into the window
template <int DEPTH, int NT>
__device__ __forceinline__ uint32_t probe_off(uint32_t base, int it, int wave, int n, uint32_t mask) {
  return (base + (uint32_t)((it * (NT / 64) + wave) * DEPTH + n) * 1024u) & mask;
}

template <int DEPTH, int NT>
__global__ __launch_bounds__(NT) void dma_probe_kernel(const char* __restrict__ g, uint32_t mask, int iters, float* out) {
  __shared__ __attribute__((aligned(1024))) char buf[64 * 1024];
  const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)buf;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t base = (blockIdx.x * 131072u) & mask;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int n = 0; n < DEPTH; ++n) {
      const uint32_t l = __builtin_amdgcn_readfirstlane(lds + (uint32_t)((wave * DEPTH + n) % 64) * 1024);
      const uint64_t src = (uint64_t)(g + probe_off<DEPTH, NT>(base, it, wave, n, mask));
      const uint64_t s = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(src >> 32)) << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)src);
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %1, %2 offset:0" ::"s"(l),
                   "v"((uint32_t)(lane * 16)), "s"((const void*)s)
                   : "memory", "m0");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = ((float*)buf)[lane];
}

template <int DEPTH, int NT>
__global__ __launch_bounds__(NT) void vgpr_probe_kernel(const char* __restrict__ g, uint32_t mask, int iters, float* out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t base = (blockIdx.x * 131072u) & mask;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
    f4 x[DEPTH];
#pragma unroll
    for (int n = 0; n < DEPTH; ++n) {
      const char* src = g + probe_off<DEPTH, NT>(base, it, wave, n, mask) + lane * 16;
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(x[n]) : "v"(src) : "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int n = 0; n < DEPTH; ++n) {
      asm volatile("" : "+v"(x[n]));  // after the wait: the loaded values are final here
      acc += x[n];
    }
  }
  if (acc[0] == 1234.5f) out[blockIdx.x] = acc[1];
}

// LDS reads: each wave keeps READS ds_read_b128 (1 KB each, conflict-free) in
// flight per batch; with DMA, each wave also issues 4 global -> LDS DMAs per
// batch into a separate 64 KB region. Per-wave clocks from s_memtime.
__device__ unsigned long long g_lds_clk[256][16];
template <int NT, int READS, bool DMA>
__global__ __launch_bounds__(NT) void lds_probe_kernel(const char* __restrict__ g, uint32_t mask, int iters, float* out) {
  __shared__ __attribute__((aligned(1024))) char buf[128 * 1024];
  const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)buf;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t rbase = lds + (uint32_t)(wave % 8) * 8192 + lane * 16;  // reads stay in the first 64 KB
  const uint32_t base = (blockIdx.x * 131072u) & mask;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    f4 x[READS];
#pragma unroll
    for (int n = 0; n < READS; ++n)
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(x[n]) : "v"(rbase), "n"((n % 8) * 1024));
    if (DMA) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const uint32_t l = __builtin_amdgcn_readfirstlane(lds + 65536u + (uint32_t)((wave * 4 + n) % 64) * 1024);
        const uint64_t src = (uint64_t)(g + ((base + (uint32_t)((it * (NT / 64) + wave) * 4 + n) * 1024u) & mask));
        const uint64_t s = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(src >> 32)) << 32) |
                           (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)src);
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %1, %2 offset:0" ::"s"(l),
                     "v"((uint32_t)(lane * 16)), "s"((const void*)s)
                     : "memory", "m0");
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int n = 0; n < READS; ++n) {
      asm volatile("" : "+v"(x[n]));
      acc += x[n];
    }
    if (DMA) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  if (lane == 0 && blockIdx.x < 256) g_lds_clk[blockIdx.x][wave] = t1 - t0;
  if (acc[0] == 1234.5f) out[blockIdx.x] = acc[1];
}

int main() {
  const uint32_t span_l2 = 2u << 20, span_hbm = 1024u << 20;
  char* g = nullptr;
  float* out = nullptr;
  if (hipMalloc(&g, (size_t)span_hbm + (1 << 20)) != hipSuccess || hipMalloc(&out, 4096 * 4) != hipSuccess) {
    fprintf(stderr, "hipMalloc failed\n");
    return 1;
  }
  (void)hipMemset(g, 1, (size_t)span_hbm + (1 << 20));
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  const int iters = 400, grid = 256;
  struct Case {
    const char* name;
    void (*k)(const char*, uint32_t, int, float*);
    int depth, nt;
  } cases[] = {{"DMA, 4 waves x 8 KB", dma_probe_kernel<8, 256>, 8, 256},
               {"DMA, 4 waves x 16 KB", dma_probe_kernel<16, 256>, 16, 256},
               {"DMA, 4 waves x 32 KB", dma_probe_kernel<32, 256>, 32, 256},
               {"DMA, 8 waves x 16 KB", dma_probe_kernel<16, 512>, 16, 512},
               {"DMA, 16 waves x 8 KB", dma_probe_kernel<8, 1024>, 8, 1024},
               {"VGPR, 4 waves x 16 KB", vgpr_probe_kernel<16, 256>, 16, 256},
               {"VGPR, 8 waves x 16 KB", vgpr_probe_kernel<16, 512>, 16, 512}};
  printf("| loads, waves per CU x bytes in flight per wave | source | GB/s per CU | GB/s total (256 CUs) |\n");
  printf("|---|---|---|---|\n");
  for (const Case& c : cases)
    for (uint32_t span : {span_l2, span_hbm}) {
      for (int w = 0; w < 3; ++w) hipLaunchKernelGGL(c.k, dim3(grid), dim3(c.nt), 0, 0, g, span - 1, iters, out);
      (void)hipEventRecord(e0);
      hipLaunchKernelGGL(c.k, dim3(grid), dim3(c.nt), 0, 0, g, span - 1, iters, out);
      (void)hipEventRecord(e1);
      if (hipEventSynchronize(e1) != hipSuccess) {
        fprintf(stderr, "kernel failed\n");
        return 1;
      }
      float ms = 0;
      (void)hipEventElapsedTime(&ms, e0, e1);
      const double bytes = (double)grid * iters * (c.nt / 64) * c.depth * 1024;
      printf("| %s | %s | %.1f | %.0f |\n", c.name, span == span_l2 ? "L2 (2 MB re-read)" : "HBM (1 GB streamed)",
             bytes / ms / 1e6 / grid, bytes / ms / 1e6);
    }

  struct LdsCase {
    const char* name;
    void (*k)(const char*, uint32_t, int, float*);
    int nt, reads;
    bool dma;
  } lcases[] = {{"4 waves, 8 reads in flight", lds_probe_kernel<256, 8, false>, 256, 8, false},
                {"4 waves, 16 reads in flight", lds_probe_kernel<256, 16, false>, 256, 16, false},
                {"8 waves, 8 reads in flight", lds_probe_kernel<512, 8, false>, 512, 8, false},
                {"4 waves, 8 reads + 4 KB of DMA per wave", lds_probe_kernel<256, 8, true>, 256, 8, true},
                {"4 waves, 16 reads + 4 KB of DMA per wave", lds_probe_kernel<256, 16, true>, 256, 16, true}};
  printf("\n| LDS: waves per CU, ds_read_b128 in flight per wave | LDS read B/clk per CU | DMA write B/clk per CU |\n");
  printf("|---|---|---|\n");
  const int lds_iters = 2000;
  for (const LdsCase& c : lcases) {
    for (int w = 0; w < 3; ++w) hipLaunchKernelGGL(c.k, dim3(grid), dim3(c.nt), 0, 0, g, span_l2 - 1, lds_iters, out);
    if (hipDeviceSynchronize() != hipSuccess) {
      fprintf(stderr, "kernel failed\n");
      return 1;
    }
    static unsigned long long clk[256][16];
    (void)hipMemcpyFromSymbol(clk, HIP_SYMBOL(g_lds_clk), sizeof(clk));
    const int nw = c.nt / 64;
    double mean = 0;
    for (int b = 0; b < grid; ++b)
      for (int w = 0; w < nw; ++w) mean += (double)clk[b][w];
    mean /= (double)grid * nw;
    const double rd = (double)lds_iters * nw * c.reads * 1024, wr = c.dma ? (double)lds_iters * nw * 4 * 1024 : 0.0;
    printf("| %s | %.1f | %.1f |\n", c.name, rd / mean, wr / mean);
  }
  return 0;
}
