// Cost of a kernel boundary on this GPU: a HIP graph of 100 back-to-back launches on one
// stream, timed with events around the graph launch (best of 5 after a warm-up), for
//   * an empty kernel in several launch shapes (1 work-group of 64 threads up to 1024
//     work-groups, with and without 128 KiB of dynamic LDS);
//   * a kernel whose 256 work-groups read what the previous launch wrote (a block written
//     by another work-group, so mostly another XCD) and write a block of the same size.
// Standalone: hipcc --offload-arch=gfx950 -O3 -o kernel_boundary kernel_boundary.hip
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

__global__ void empty_kernel(int* p) {
  if (p == nullptr && threadIdx.x == 1000) p[0] = 1;  // never true: keeps the argument
}

// reads block (blockIdx + 37) % grid of src, writes block blockIdx of dst (vec 16-byte words each)
__global__ __launch_bounds__(512) void chain_kernel(const u32x4* src, u32x4* dst, int vec) {
  const int rb = (blockIdx.x + 37) % gridDim.x;
  for (int i = threadIdx.x; i < vec; i += blockDim.x) {
    u32x4 v = src[(long)rb * vec + i];
    v.x += 1;
    dst[(long)blockIdx.x * vec + i] = v;
  }
}

struct Case {
  const char* name;
  int grid, block, lds, chain_vec;  // chain_vec 0: empty kernel
};

int main() {
  const int n = 100, max_grid = 1024, max_vec = 8192 / 16;
  u32x4 *a, *b;
  CHECK(hipMalloc(&a, (size_t)max_grid * max_vec * 16));
  CHECK(hipMalloc(&b, (size_t)max_grid * max_vec * 16));
  CHECK(hipMemset(a, 0, (size_t)max_grid * max_vec * 16));
  CHECK(hipMemset(b, 0, (size_t)max_grid * max_vec * 16));
  CHECK(hipFuncSetAttribute((const void*)empty_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 131072));
  hipStream_t s;
  CHECK(hipStreamCreate(&s));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const Case cases[] = {
      {"empty, 1 work-group x 64", 1, 64, 0, 0},
      {"empty, 256 work-groups x 64", 256, 64, 0, 0},
      {"empty, 256 work-groups x 512", 256, 512, 0, 0},
      {"empty, 256 work-groups x 512, 128 KiB LDS", 256, 512, 131072, 0},
      {"empty, 1024 work-groups x 256", 1024, 256, 0, 0},
      {"read + write 1 KiB per work-group, 256 x 512", 256, 512, 0, 64},
      {"read + write 8 KiB per work-group, 256 x 512", 256, 512, 0, 512},
  };
  for (const Case& c : cases) {
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    for (int i = 0; i < n; ++i) {
      if (c.chain_vec == 0) {
        hipLaunchKernelGGL(empty_kernel, dim3(c.grid), dim3(c.block), c.lds, s, (int*)a);
      } else {
        hipLaunchKernelGGL(chain_kernel, dim3(c.grid), dim3(c.block), 0, s, (i & 1) ? b : a, (i & 1) ? a : b,
                           c.chain_vec);
      }
    }
    CHECK(hipStreamEndCapture(s, &g));
    CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    float best = 1e9f;
    for (int r = 0; r < 6; ++r) {
      CHECK(hipEventRecord(e0, s));
      CHECK(hipGraphLaunch(ge, s));
      CHECK(hipEventRecord(e1, s));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      if (r > 0 && ms < best) best = ms;
    }
    printf("%-50s %6.2f us per kernel\n", c.name, best * 1e3f / n);
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
  }
  CHECK(hipDeviceSynchronize());
  return 0;
}
