// Bytes a CU can pull in: 256 work-groups of 8 waves (one per CU) stream 64 KiB per
// iteration each, two iterations in flight, either by LDS DMA (global_load_lds_dwordx4
// into a 2 x 64 KiB LDS ring, the copy path of the attention, projection and LM-head
// kernels) or by global_load_dwordx4 into registers, from
//   * one region every work-group reads (256 KiB or 640 KiB: L2-resident, the way the
//     GEMMs re-read their activation rows), in step or with the work-groups of an XCD
//     starting at different offsets;
//   * a private 4 MiB region per work-group (1 GiB from HBM).
// Standalone: hipcc --offload-arch=gfx950 -O3 -o cu_ingest cu_ingest.hip
#include <hip/hip_runtime.h>
#include <cstdio>

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));             \
      return 1;                                                           \
    }                                                                     \
  } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void lds_dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// iteration it: wave w copies KiB (64 it + 8 j + w) mod region for j < 8 into LDS slot it & 1
__global__ __launch_bounds__(512) void dma_stream(const char* src, long region, long per_wg, int iters, int stagger,
                                                  int* sink) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const char* base = src + per_wg * blockIdx.x;
  const int start = stagger ? ((blockIdx.x / 8) % 8) * 4 : 0;  // work-groups b and b + 8 share an XCD
  for (int it = 0; it < iters; ++it) {
    char* slot = lds + (it & 1) * 65536;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const long off = ((long)((it + start) * 64 + j * 8 + wave) * 1024) % region + lane * 16;
      lds_dma16(base + off, slot + (j * 8 + wave) * 1024);
    }
    if (it > 0) wait_vm<8>();  // iteration it - 1 has landed
    __syncthreads();
  }
  wait_vm<0>();  // no copy may land after the work-group has left
  __syncthreads();
  if (threadIdx.x == 0 && lds[5] == 123 && lds[70000] == 45) sink[blockIdx.x] = 1;
}

__global__ __launch_bounds__(512) void vgpr_stream(const char* src, long region, long per_wg, int iters, int* sink) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const char* base = src + per_wg * blockIdx.x;
  auto at = [&](int it, int j) { return (const u32x4*)(base + ((long)(it * 64 + j * 8 + wave) * 1024) % region + lane * 16); };
  u32x4 acc = {0, 0, 0, 0}, a[8], b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = *at(0, j);
  for (int it = 1; it < iters; it += 2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = *at(it, j);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= a[j];
    if (it + 1 < iters) {
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = *at(it + 1, j);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= b[j];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x12345678u) sink[blockIdx.x * 512 + threadIdx.x] = 1;
}

struct Case {
  const char* name;
  long region, per_wg;
  int iters;
};

int main() {
  const int grid = 256;
  const long hbm_per_wg = 4l << 20;
  char* buf;
  int* sink;
  CHECK(hipMalloc(&buf, hbm_per_wg * grid));
  CHECK(hipMalloc(&sink, grid * 512 * sizeof(int)));
  CHECK(hipMemset(buf, 1, hbm_per_wg * grid));
  CHECK(hipFuncSetAttribute((const void*)dma_stream, hipFuncAttributeMaxDynamicSharedMemorySize, 131072));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const Case cases[] = {{"shared 256 KiB (L2)", 256 << 10, 0, 256},
                        {"shared 640 KiB (L2)", 640 << 10, 0, 256},
                        {"private 4 MiB per work-group (HBM)", hbm_per_wg, hbm_per_wg, 64}};
  const char* kinds[] = {"LDS DMA", "LDS DMA, staggered", "global_load into VGPRs"};
  for (int rep = 0; rep < 2; ++rep) {  // the first pass warms clocks and caches
    for (const Case& c : cases) {
      for (int kind = 0; kind < 3; ++kind) {
        float best = 1e9f;
        for (int r = 0; r < 5; ++r) {
          CHECK(hipEventRecord(e0));
          if (kind < 2) {
            hipLaunchKernelGGL(dma_stream, dim3(grid), dim3(512), 131072, 0, buf, c.region, c.per_wg, c.iters,
                               kind, sink);
          } else {
            hipLaunchKernelGGL(vgpr_stream, dim3(grid), dim3(512), 0, 0, buf, c.region, c.per_wg, c.iters, sink);
          }
          CHECK(hipEventRecord(e1));
          CHECK(hipEventSynchronize(e1));
          float ms;
          CHECK(hipEventElapsedTime(&ms, e0, e1));
          if (ms < best) best = ms;
        }
        const double bytes = (double)grid * c.iters * 65536;
        if (rep == 1)
          printf("%-36s %-24s %8.1f us  %6.2f TB/s  %5.1f GB/s per CU\n", c.name, kinds[kind], best * 1e3f,
                 bytes / best / 1e9, bytes / best / 1e6 / grid);
      }
    }
  }
  CHECK(hipDeviceSynchronize());
  return 0;
}
