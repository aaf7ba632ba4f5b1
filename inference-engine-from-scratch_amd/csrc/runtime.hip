// Library-level pieces of libnanoengine_hip: per-thread error text, launch
// checking, ABI version and a plain copy kernel used to calibrate the hardware
// byte counters (FETCH_SIZE / WRITE_SIZE) against a kernel of known traffic.
#include <stdarg.h>

#include "ne_common.hpp"

namespace ne {

namespace {
thread_local char g_error[512] = "";

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* src, u32x4* dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = src[i];
}
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return NE_ELAUNCH;
  }
  return NE_OK;
}

}  // namespace ne

extern "C" int ne_abi_version(void) { return NE_ABI_VERSION; }

extern "C" const char* ne_last_error(void) { return ne::g_error; }

extern "C" int ne_copy_bytes(const void* src, void* dst, size_t bytes, void* stream) {
  NE_CHECK_ARG(src && dst, "null pointer argument");
  NE_CHECK_ARG(bytes % 16 == 0, "bytes must be a multiple of 16");
  NE_CHECK_ARG(((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0,
               "src and dst must be 16-byte aligned");
  if (bytes == 0) return NE_OK;
  const int64_t n = (int64_t)(bytes / 16);
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 256 * 8);
  hipLaunchKernelGGL(ne::copy_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     (const ne::u32x4*)src, (ne::u32x4*)dst, n);
  return ne::check_launch("copy_bytes");
}
