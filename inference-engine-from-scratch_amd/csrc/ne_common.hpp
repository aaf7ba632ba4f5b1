// Shared device types, launch helpers and error reporting for libnanoengine_hip.
// Target: gfx950 only (64-wide waves, bf16/f16 MFMA, 160 KB LDS per CU).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "nanoengine_hip.h"

namespace ne {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// int32 read through the scalar cache: loads of a wave-uniform address in the constant
// address space compile to s_load (data written by an earlier kernel only)
using ConstI32 = __attribute__((address_space(4))) const int32_t;

constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, work-groups dispatched round-robin

// ---- error state (per calling thread) ------------------------------------
void set_error(const char* fmt, ...);

#define NE_CHECK_ARG(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      ::ne::set_error(__VA_ARGS__);          \
      return NE_EINVAL;                      \
    }                                        \
  } while (0)

#define NE_CHECK_SUPPORTED(cond, ...)        \
  do {                                       \
    if (!(cond)) {                           \
      ::ne::set_error(__VA_ARGS__);          \
      return NE_EUNSUPPORTED;                \
    }                                        \
  } while (0)

int check_launch(const char* what);

// ---- numeric helpers ------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// round-to-nearest-even f32 -> bf16 (finite inputs; NaN stays NaN)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// two f32 -> packed bf16 pair (lo in bits 0..15), one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  floatx2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// scale element of dtype NE_DTYPE_{BF16,FP16,FP32} at index i
template <int DT>
__device__ __forceinline__ float load_scale(const void* p, int64_t i) {
  if constexpr (DT == NE_DTYPE_BF16) {
    return bf16_to_f32(((const uint16_t*)p)[i]);
  } else if constexpr (DT == NE_DTYPE_FP16) {
    return f16_to_f32(((const uint16_t*)p)[i]);
  } else {
    return ((const float*)p)[i];
  }
}

template <int DT>
__device__ __forceinline__ void store_scale(void* p, int64_t i, float v) {
  if constexpr (DT == NE_DTYPE_BF16) {
    ((uint16_t*)p)[i] = f32_to_bf16(v);
  } else if constexpr (DT == NE_DTYPE_FP16) {
    ((uint16_t*)p)[i] = f32_to_f16(v);
  } else {
    ((float*)p)[i] = v;
  }
}

// Work-group barrier ordering LDS accesses only: waits for this wave's LDS operations,
// not for its global loads in flight (a __syncthreads fence would wait for those too).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // lgkmcnt(0), vmcnt / expcnt left alone
  __asm__ __volatile__("s_barrier" ::: "memory");
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace ne
