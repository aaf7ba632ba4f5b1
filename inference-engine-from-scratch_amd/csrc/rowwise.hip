// Row-wise kernels of the Qwen3 verify forward for gfx950: RMSNorm (plain,
// fused with the residual add, fused with the embedding gather), the fused
// QK-norm + RoPE + KV-cache write, and the standalone KV write/quantise.
//
// Rounding follows the reference's bf16 op sequence so results stay within
// bf16 noise of it:
//   RMSNorm (ne/models/qwen3.py:39-44): h32 = fp32(x); bf16(h32 * rsqrt(mean(h32^2)+eps))
//            then bf16(weight * that)
//   RoPE    (ne/models/qwen3.py:47-68): cos/sin of fp32 angle pos*inv_freq rounded to
//            bf16; bf16(bf16(x*cos) + bf16(rotate_half(x)*sin))
//   int8 KV (ne/models/int8_quantization.py:30-34): s = max(amax, 1e-8)/127 in fp32,
//            code = rint(fp32(x)/s) clamped to +-127, stored scale = s in the scale dtype
#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kMaxChunksPerLane = 8;  // hidden <= 64 lanes * 8 chunks * 8 = 4096

__device__ __forceinline__ void unpack8(const u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_to_f32((uint16_t)(v[i] & 0xFFFFu));
    f[2 * i + 1] = bf16_to_f32((uint16_t)(v[i] >> 16));
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
               pack_bf16x2(f[6], f[7])};
}

// MODE 0: out = norm(x); 1: residual = bf16(residual + delta), out = norm(residual);
// 2: residual = embed[token], out = norm(residual); 3: as 1 with
// delta = bf16(sum over `splits` fp32 partial rows, split stride rows * hidden).
// One wave per row.
template <int MODE>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, uint16_t* residual,
                                                      const uint16_t* delta, const int32_t* tokens,
                                                      const uint16_t* embed, const uint16_t* weight,
                                                      uint16_t* out, int rows, int hidden,
                                                      float eps, const float* partials = nullptr,
                                                      int splits = 0) {
  const int row = blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const int chunks = hidden / 8;
  const uint16_t* src;
  if constexpr (MODE == 0) {
    src = x + (int64_t)row * hidden;
  } else if constexpr (MODE == 1 || MODE == 3) {
    src = residual + (int64_t)row * hidden;
  } else {
    src = embed + (int64_t)tokens[row] * hidden;
  }
  float h[kMaxChunksPerLane][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ci = lane + c * kWave;
    if (ci < chunks) {
      unpack8(*(const u32x4*)(src + ci * 8), h[c]);
      if constexpr (MODE == 1) {
        float d[8];
        unpack8(*(const u32x4*)(delta + (int64_t)row * hidden + ci * 8), d);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[c][e] = bf16_round(h[c][e] + d[e]);
      } else if constexpr (MODE == 3) {
        float d[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < splits; ++sp) {
          const float* pp = partials + ((int64_t)sp * rows + row) * hidden + ci * 8;
          const floatx4 lo = *(const floatx4*)pp;
          const floatx4 hi = *(const floatx4*)(pp + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            d[e] += lo[e];
            d[e + 4] += hi[e];
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) h[c][e] = bf16_round(h[c][e] + bf16_round(d[e]));
      }
      if constexpr (MODE != 0) *(u32x4*)(residual + (int64_t)row * hidden + ci * 8) = pack8(h[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += h[c][e] * h[c][e];
    }
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ci = lane + c * kWave;
    if (ci < chunks) {
      float w[8], o[8];
      unpack8(*(const u32x4*)(weight + ci * 8), w);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = bf16_round(h[c][e] * inv) * w[e];
      *(u32x4*)(out + (int64_t)row * hidden + ci * 8) = pack8(o);
    }
  }
}

// Quantise (int8 cache) or copy one 128-vector held as lane / lane+64 values.
template <bool INT8, int SDT>
__device__ __forceinline__ void write_vector(float a, float b, int lane, int64_t slot, int head,
                                             int num_heads, void* cache, void* scales) {
  const int64_t base = (slot * num_heads + head) * 128;
  if constexpr (INT8) {
    float amax = fmaxf(fabsf(a), fabsf(b));
    amax = wave_max(amax);
    const float s = fmaxf(amax, 1e-8f) / 127.f;
    const float qa = fminf(fmaxf(rintf(a / s), -127.f), 127.f);
    const float qb = fminf(fmaxf(rintf(b / s), -127.f), 127.f);
    int8_t* c = (int8_t*)cache + base;
    c[lane] = (int8_t)(int)qa;
    c[lane + 64] = (int8_t)(int)qb;
    if (lane == 0) store_scale<SDT>(scales, slot * num_heads + head, s);
  } else {
    uint16_t* c = (uint16_t*)cache + base;
    c[lane] = f32_to_bf16(a);
    c[lane + 64] = f32_to_bf16(b);
  }
}

// One 256-thread work-group per token row; waves walk q heads, then k heads, then v heads.
template <bool INT8, int SDT>
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(
    const uint16_t* qkv, int hq, int hkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
    float eps, const int32_t* positions, const float* inv_freq, const int32_t* slot_mapping,
    void* k_cache, void* v_cache, void* k_scale, void* v_scale, uint16_t* q_out) {
  const int row = blockIdx.x;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int width = (hq + 2 * hkv) * 128;
  const uint16_t* src = qkv + (int64_t)row * width;
  const float pos = (float)positions[row];
  const int64_t slot = slot_mapping[row];
  // rotary factors for dims lane and lane+64 share one angle
  float sn, cs;
  sincosf(pos * inv_freq[lane], &sn, &cs);
  const float c16 = bf16_round(cs), s16 = bf16_round(sn);
  for (int h = wave; h < hq + 2 * hkv; h += 4) {
    const uint16_t* v = src + h * 128;
    float a = bf16_to_f32(v[lane]);
    float b = bf16_to_f32(v[lane + 64]);
    if (h < hq + hkv) {
      const uint16_t* w = (h < hq) ? q_norm_w : k_norm_w;
      const float inv = rsqrtf(wave_sum(a * a + b * b) / 128.f + eps);
      a = bf16_round(bf16_round(a * inv) * bf16_to_f32(w[lane]));
      b = bf16_round(bf16_round(b * inv) * bf16_to_f32(w[lane + 64]));
      const float ra = bf16_round(bf16_round(a * c16) + bf16_round(-b * s16));
      const float rb = bf16_round(bf16_round(b * c16) + bf16_round(a * s16));
      if (h < hq) {
        uint16_t* qo = q_out + ((int64_t)row * hq + h) * 128;
        qo[lane] = f32_to_bf16(ra);
        qo[lane + 64] = f32_to_bf16(rb);
      } else {
        write_vector<INT8, SDT>(ra, rb, lane, slot, h - hq, hkv, k_cache, k_scale);
      }
    } else {
      write_vector<INT8, SDT>(a, b, lane, slot, h - hq - hkv, hkv, v_cache, v_scale);
    }
  }
}

// Standalone A7: vectors [n, heads, 128] -> cache at slot_mapping, one wave per vector.
template <bool INT8, int VDT, int SDT>
__global__ __launch_bounds__(256) void kv_write_kernel(const uint16_t* vectors, int64_t n,
                                                       int heads, const int32_t* slot_mapping,
                                                       void* cache, void* scales) {
  const int64_t vec = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (vec >= n * heads) return;
  const int64_t row = vec / heads;
  const int head = (int)(vec % heads);
  const uint16_t* v = vectors + vec * 128;
  float a, b;
  if constexpr (VDT == NE_DTYPE_FP16) {
    a = f16_to_f32(v[lane]);
    b = f16_to_f32(v[lane + 64]);
  } else {
    a = bf16_to_f32(v[lane]);
    b = bf16_to_f32(v[lane + 64]);
  }
  const int64_t slot = slot_mapping[row];
  if constexpr (INT8) {
    write_vector<true, SDT>(a, b, lane, slot, head, heads, cache, scales);
  } else {
    // plain scatter keeps the exact input bits
    uint16_t* c = (uint16_t*)cache + (slot * heads + head) * 128;
    c[lane] = v[lane];
    c[lane + 64] = v[lane + 64];
  }
}

}  // namespace

}  // namespace ne

using namespace ne;

static int check_norm_args(const void* weight, const void* out, int32_t rows, int32_t hidden) {
  NE_CHECK_ARG(rows >= 0, "rows < 0");
  NE_CHECK_ARG(weight && out, "null pointer argument");
  NE_CHECK_SUPPORTED(hidden > 0 && hidden % 8 == 0 && hidden <= kWave * kMaxChunksPerLane * 8,
                     "hidden must be a multiple of 8 and <= %d (got %d)",
                     kWave * kMaxChunksPerLane * 8, hidden);
  return NE_OK;
}

extern "C" int ne_rmsnorm(const void* x, const void* weight, void* out, int32_t rows,
                          int32_t hidden, float eps, void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(x != nullptr, "null x");
  if (rows == 0) return NE_OK;
  hipLaunchKernelGGL(rmsnorm_kernel<0>, dim3(ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, nullptr, nullptr, nullptr, nullptr,
                     (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps);
  return check_launch("rmsnorm");
}

extern "C" int ne_add_rmsnorm(void* residual, const void* delta, const void* weight, void* out,
                              int32_t rows, int32_t hidden, float eps, void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(residual && delta, "null residual/delta");
  if (rows == 0) return NE_OK;
  hipLaunchKernelGGL(rmsnorm_kernel<1>, dim3(ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                     nullptr, (uint16_t*)residual, (const uint16_t*)delta, nullptr, nullptr,
                     (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps);
  return check_launch("add_rmsnorm");
}

extern "C" int ne_splitk_add_rmsnorm(void* residual, const float* partials, int32_t splits,
                                     const void* weight, void* out, int32_t rows, int32_t hidden,
                                     float eps, void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(residual && partials, "null residual/partials");
  NE_CHECK_ARG(splits >= 1 && splits <= 64, "splits must be in [1, 64] (got %d)", splits);
  NE_CHECK_ARG(((uintptr_t)partials % 16) == 0, "partials must be 16-byte aligned");
  if (rows == 0) return NE_OK;
  hipLaunchKernelGGL(rmsnorm_kernel<3>, dim3(ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                     nullptr, (uint16_t*)residual, nullptr, nullptr, nullptr,
                     (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps, partials, splits);
  return check_launch("splitk_add_rmsnorm");
}

extern "C" int ne_embed_rmsnorm(const int32_t* tokens, const void* embed, const void* weight,
                                void* residual, void* out, int32_t rows, int32_t hidden, float eps,
                                void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(tokens && embed && residual, "null tokens/embed/residual");
  if (rows == 0) return NE_OK;
  hipLaunchKernelGGL(rmsnorm_kernel<2>, dim3(ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                     nullptr, (uint16_t*)residual, nullptr, tokens, (const uint16_t*)embed,
                     (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps);
  return check_launch("embed_rmsnorm");
}

extern "C" int ne_qk_norm_rope_kv_write(const void* qkv, int32_t rows, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        const void* q_norm_weight, const void* k_norm_weight,
                                        float eps, const int32_t* positions,
                                        const float* inv_freq, const int32_t* slot_mapping,
                                        void* k_cache, void* v_cache, void* k_scale,
                                        void* v_scale, int32_t kv_dtype, int32_t scale_dtype,
                                        void* q_out, void* stream) {
  NE_CHECK_ARG(rows >= 0, "rows < 0");
  if (rows == 0) return NE_OK;
  NE_CHECK_SUPPORTED(head_dim == 128, "head_dim must be 128 (got %d)", head_dim);
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0, "bad head counts");
  NE_CHECK_ARG(qkv && q_norm_weight && k_norm_weight && positions && inv_freq && slot_mapping &&
                   k_cache && v_cache && q_out,
               "null pointer argument");
  NE_CHECK_ARG(kv_dtype == NE_DTYPE_BF16 || kv_dtype == NE_DTYPE_INT8,
               "kv_dtype must be bf16 or int8");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(rows), block(256);
#define NE_QKR_ARGS                                                                              \
  (const uint16_t*)qkv, num_q_heads, num_kv_heads, (const uint16_t*)q_norm_weight,              \
      (const uint16_t*)k_norm_weight, eps, positions, inv_freq, slot_mapping, k_cache, v_cache, \
      k_scale, v_scale, (uint16_t*)q_out
  if (kv_dtype == NE_DTYPE_BF16) {
    hipLaunchKernelGGL((qk_norm_rope_kv_kernel<false, NE_DTYPE_BF16>), grid, block, 0, s,
                       NE_QKR_ARGS);
  } else {
    NE_CHECK_ARG(k_scale && v_scale, "int8 cache needs scales");
    if (scale_dtype == NE_DTYPE_BF16) {
      hipLaunchKernelGGL((qk_norm_rope_kv_kernel<true, NE_DTYPE_BF16>), grid, block, 0, s,
                         NE_QKR_ARGS);
    } else if (scale_dtype == NE_DTYPE_FP16) {
      hipLaunchKernelGGL((qk_norm_rope_kv_kernel<true, NE_DTYPE_FP16>), grid, block, 0, s,
                         NE_QKR_ARGS);
    } else if (scale_dtype == NE_DTYPE_FP32) {
      hipLaunchKernelGGL((qk_norm_rope_kv_kernel<true, NE_DTYPE_FP32>), grid, block, 0, s,
                         NE_QKR_ARGS);
    } else {
      set_error("scale_dtype must be bf16, fp16 or fp32");
      return NE_EINVAL;
    }
  }
#undef NE_QKR_ARGS
  return check_launch("qk_norm_rope_kv_write");
}

extern "C" int ne_kv_write(const void* vectors, int32_t vec_dtype, int64_t n, int32_t num_heads,
                           int32_t head_dim, const int32_t* slot_mapping, void* cache,
                           int32_t cache_dtype, void* scales, int32_t scale_dtype, void* stream) {
  NE_CHECK_ARG(n >= 0 && num_heads > 0, "bad shape");
  if (n == 0) return NE_OK;
  NE_CHECK_SUPPORTED(head_dim == 128, "head_dim must be 128 (got %d)", head_dim);
  NE_CHECK_ARG(vectors && slot_mapping && cache, "null pointer argument");
  NE_CHECK_ARG(vec_dtype == NE_DTYPE_BF16 || vec_dtype == NE_DTYPE_FP16,
               "vectors must be bf16 or fp16");
  NE_CHECK_ARG(cache_dtype == NE_DTYPE_INT8 || cache_dtype == vec_dtype,
               "cache dtype must be int8 or equal to the vector dtype");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)ceil_div(n * num_heads, 4)), block(256);
  const uint16_t* v = (const uint16_t*)vectors;
  if (cache_dtype != NE_DTYPE_INT8) {
    hipLaunchKernelGGL((kv_write_kernel<false, NE_DTYPE_BF16, NE_DTYPE_BF16>), grid, block, 0, s,
                       v, n, num_heads, slot_mapping, cache, scales);
    return check_launch("kv_write");
  }
  NE_CHECK_ARG(scales != nullptr, "int8 cache needs scales");
#define NE_KVW(VDT, SDT)                                                                       \
  hipLaunchKernelGGL((kv_write_kernel<true, VDT, SDT>), grid, block, 0, s, v, n, num_heads,   \
                     slot_mapping, cache, scales)
  if (vec_dtype == NE_DTYPE_BF16) {
    if (scale_dtype == NE_DTYPE_BF16) NE_KVW(NE_DTYPE_BF16, NE_DTYPE_BF16);
    else if (scale_dtype == NE_DTYPE_FP16) NE_KVW(NE_DTYPE_BF16, NE_DTYPE_FP16);
    else if (scale_dtype == NE_DTYPE_FP32) NE_KVW(NE_DTYPE_BF16, NE_DTYPE_FP32);
    else { set_error("bad scale_dtype"); return NE_EINVAL; }
  } else {
    if (scale_dtype == NE_DTYPE_BF16) NE_KVW(NE_DTYPE_FP16, NE_DTYPE_BF16);
    else if (scale_dtype == NE_DTYPE_FP16) NE_KVW(NE_DTYPE_FP16, NE_DTYPE_FP16);
    else if (scale_dtype == NE_DTYPE_FP32) NE_KVW(NE_DTYPE_FP16, NE_DTYPE_FP32);
    else { set_error("bad scale_dtype"); return NE_EINVAL; }
  }
#undef NE_KVW
  return check_launch("kv_write");
}
