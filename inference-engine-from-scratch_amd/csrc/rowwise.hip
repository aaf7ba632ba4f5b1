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
#include "qk_rope_kv.hpp"

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
// delta = bf16(sum over SPLITS fp32 partial rows, split stride rows * hidden).
// One wave per row.  Every load of a row (input, delta or partials, weight) is
// issued before the first use, so a wave pays one memory round trip, not one per
// split: SPLITS is a template parameter for that reason, and so is CPL, the 8-element
// chunks per lane (hidden <= 512 * CPL), which sizes the register arrays.
template <int MODE, int SPLITS, int CPL>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, uint16_t* residual,
                                                      const uint16_t* delta, const int32_t* tokens,
                                                      const uint16_t* embed, const uint16_t* weight,
                                                      uint16_t* out, int rows, int hidden,
                                                      float eps, const float* partials = nullptr) {
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
  u32x4 raw[CPL], wraw[CPL], draw[CPL];
  floatx4 part[CPL][SPLITS > 0 ? SPLITS : 1][2];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ci = lane + c * kWave;
    if (ci < chunks) {
      raw[c] = *(const u32x4*)(src + ci * 8);
      wraw[c] = *(const u32x4*)(weight + ci * 8);
      if constexpr (MODE == 1) draw[c] = *(const u32x4*)(delta + (int64_t)row * hidden + ci * 8);
      if constexpr (MODE == 3) {
#pragma unroll
        for (int sp = 0; sp < SPLITS; ++sp) {
          const float* pp = partials + ((int64_t)sp * rows + row) * hidden + ci * 8;
          part[c][sp][0] = *(const floatx4*)pp;
          part[c][sp][1] = *(const floatx4*)(pp + 4);
        }
      }
    }
  }
  float h[CPL][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ci = lane + c * kWave;
    if (ci < chunks) {
      unpack8(raw[c], h[c]);
      if constexpr (MODE == 1) {
        float d[8];
        unpack8(draw[c], d);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[c][e] = bf16_round(h[c][e] + d[e]);
      } else if constexpr (MODE == 3) {
        float d[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < SPLITS; ++sp) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            d[e] += part[c][sp][0][e];
            d[e + 4] += part[c][sp][1][e];
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
  for (int c = 0; c < CPL; ++c) {
    const int ci = lane + c * kWave;
    if (ci < chunks) {
      float w[8], o[8];
      unpack8(wraw[c], w);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = bf16_round(h[c][e] * inv) * w[e];
      *(u32x4*)(out + (int64_t)row * hidden + ci * 8) = pack8(o);
    }
  }
}

// One wave per (token row, head), four heads of a row per work-group: q heads,
// then k heads, then v heads.  cos/sin come from `rope` ([rope_positions][2][64]
// bf16: cos, then sin, of position * inv_freq[i]; dims i and i + 64 share them),
// computed once by the caller exactly as the reference builds its tables.
template <bool INT8, int SDT>
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(
    const uint16_t* qkv, int hq, int hkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
    float eps, const int32_t* positions, const uint16_t* rope, int rope_positions,
    const int32_t* slot_mapping, void* k_cache, void* v_cache, void* k_scale, void* v_scale,
    uint16_t* q_out) {
  const int heads = hq + 2 * hkv;
  const int groups = (heads + 3) / 4;
  const int row = blockIdx.x / groups;
  const int h = (blockIdx.x % groups) * 4 + threadIdx.x / kWave;
  if (h >= heads) return;  // wave-uniform; the kernel has no barrier
  const int lane = threadIdx.x % kWave;
  const uint16_t* v = qkv + (int64_t)row * heads * 128 + h * 128;
  const float a = bf16_to_f32(v[lane]);
  const float b = bf16_to_f32(v[lane + 64]);
  const int64_t slot = slot_mapping[row];
  float wa = 0.f, wb = 0.f, c16 = 0.f, s16 = 0.f;
  if (h < hq + hkv) {
    const uint16_t* w = (h < hq) ? q_norm_w : k_norm_w;
    wa = bf16_to_f32(w[lane]);
    wb = bf16_to_f32(w[lane + 64]);
    const int pos = min(max(positions[row], 0), rope_positions - 1);
    c16 = bf16_to_f32(rope[(int64_t)pos * 128 + lane]);
    s16 = bf16_to_f32(rope[(int64_t)pos * 128 + 64 + lane]);
  }
  const QkvRopeArgs q{hq, hkv, q_norm_w, k_norm_w, eps, positions, rope, rope_positions, slot_mapping,
                      k_cache, v_cache, k_scale, v_scale, q_out};
  const int rows1[1] = {row};
  const bool valid1[1] = {true};
  float av[1] = {a}, bv[1] = {b};
  const int64_t sv[1] = {slot};
  const float cv[1] = {c16}, sn[1] = {s16};
  qk_norm_rope_kv_vectors<INT8, SDT, 1>(q, rows1, valid1, h, lane, av, bv, sv, wa, wb, cv, sn);
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

// 8-element chunks per lane for a row of `hidden` elements (one wave per row)
static int chunks_per_lane(int hidden) { return hidden <= 1024 ? 2 : hidden <= 2048 ? 4 : 8; }

#define NE_NORM_LAUNCH(MODE, SPLITS, ...)                                                     \
  do {                                                                                         \
    const int cpl = chunks_per_lane(hidden);                                                   \
    if (cpl == 2)                                                                              \
      hipLaunchKernelGGL((rmsnorm_kernel<MODE, SPLITS, 2>), grid, block, 0, s, __VA_ARGS__);   \
    else if (cpl == 4)                                                                         \
      hipLaunchKernelGGL((rmsnorm_kernel<MODE, SPLITS, 4>), grid, block, 0, s, __VA_ARGS__);   \
    else                                                                                       \
      hipLaunchKernelGGL((rmsnorm_kernel<MODE, SPLITS, 8>), grid, block, 0, s, __VA_ARGS__);   \
  } while (0)

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
  const dim3 grid(ceil_div(rows, 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  NE_NORM_LAUNCH(0, 0, (const uint16_t*)x, nullptr, nullptr, nullptr, nullptr,
                 (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps, nullptr);
  return check_launch("rmsnorm");
}

extern "C" int ne_add_rmsnorm(void* residual, const void* delta, const void* weight, void* out,
                              int32_t rows, int32_t hidden, float eps, void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(residual && delta, "null residual/delta");
  if (rows == 0) return NE_OK;
  const dim3 grid(ceil_div(rows, 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  NE_NORM_LAUNCH(1, 0, nullptr, (uint16_t*)residual, (const uint16_t*)delta, nullptr, nullptr,
                 (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps, nullptr);
  return check_launch("add_rmsnorm");
}

extern "C" int ne_splitk_add_rmsnorm(void* residual, const float* partials, int32_t splits,
                                     const void* weight, void* out, int32_t rows, int32_t hidden,
                                     float eps, void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(residual && partials, "null residual/partials");
  NE_CHECK_ARG(splits >= 1, "splits must be >= 1 (got %d)", splits);
  NE_CHECK_ARG(((uintptr_t)partials % 16) == 0, "partials must be 16-byte aligned");
  if (rows == 0) return NE_OK;
  const dim3 grid(ceil_div(rows, 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  // the partials of SPLITS x CPL chunks stay in registers: keep that product small
  NE_CHECK_SUPPORTED(splits * chunks_per_lane(hidden) <= 16,
                     "splits x hidden too large for the fused split-K norm (splits=%d, hidden=%d)",
                     splits, hidden);
#define NE_SPLITK_NORM(S, C)                                                                  \
  hipLaunchKernelGGL((rmsnorm_kernel<3, S, C>), grid, block, 0, s, nullptr, (uint16_t*)residual, \
                     nullptr, nullptr, nullptr, (const uint16_t*)weight, (uint16_t*)out, rows,    \
                     hidden, eps, partials)
  const int cpl = chunks_per_lane(hidden);
  switch (splits * 16 + cpl) {
    case 1 * 16 + 2: NE_SPLITK_NORM(1, 2); break;
    case 2 * 16 + 2: NE_SPLITK_NORM(2, 2); break;
    case 3 * 16 + 2: NE_SPLITK_NORM(3, 2); break;
    case 4 * 16 + 2: NE_SPLITK_NORM(4, 2); break;
    case 6 * 16 + 2: NE_SPLITK_NORM(6, 2); break;
    case 8 * 16 + 2: NE_SPLITK_NORM(8, 2); break;
    case 1 * 16 + 4: NE_SPLITK_NORM(1, 4); break;
    case 2 * 16 + 4: NE_SPLITK_NORM(2, 4); break;
    case 3 * 16 + 4: NE_SPLITK_NORM(3, 4); break;
    case 4 * 16 + 4: NE_SPLITK_NORM(4, 4); break;
    case 1 * 16 + 8: NE_SPLITK_NORM(1, 8); break;
    case 2 * 16 + 8: NE_SPLITK_NORM(2, 8); break;
    default:
      set_error("splits must be 1, 2, 3, 4, 6 or 8 (got %d)", splits);
      return NE_EUNSUPPORTED;
  }
#undef NE_SPLITK_NORM
  return check_launch("splitk_add_rmsnorm");
}

extern "C" int ne_embed_rmsnorm(const int32_t* tokens, const void* embed, const void* weight,
                                void* residual, void* out, int32_t rows, int32_t hidden, float eps,
                                void* stream) {
  int rc = check_norm_args(weight, out, rows, hidden);
  if (rc != NE_OK) return rc;
  NE_CHECK_ARG(tokens && embed && residual, "null tokens/embed/residual");
  if (rows == 0) return NE_OK;
  const dim3 grid(ceil_div(rows, 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  NE_NORM_LAUNCH(2, 0, nullptr, (uint16_t*)residual, nullptr, tokens, (const uint16_t*)embed,
                 (const uint16_t*)weight, (uint16_t*)out, rows, hidden, eps, nullptr);
  return check_launch("embed_rmsnorm");
}

extern "C" int ne_qk_norm_rope_kv_write(const void* qkv, int32_t rows, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        const void* q_norm_weight, const void* k_norm_weight,
                                        float eps, const int32_t* positions,
                                        const void* rope_cos_sin, int32_t rope_positions,
                                        const int32_t* slot_mapping,
                                        void* k_cache, void* v_cache, void* k_scale,
                                        void* v_scale, int32_t kv_dtype, int32_t scale_dtype,
                                        void* q_out, void* stream) {
  NE_CHECK_ARG(rows >= 0, "rows < 0");
  if (rows == 0) return NE_OK;
  NE_CHECK_SUPPORTED(head_dim == 128, "head_dim must be 128 (got %d)", head_dim);
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0, "bad head counts");
  NE_CHECK_ARG(qkv && q_norm_weight && k_norm_weight && positions && rope_cos_sin && slot_mapping &&
                   k_cache && v_cache && q_out,
               "null pointer argument");
  NE_CHECK_ARG(rope_positions > 0, "rope_positions must be positive");
  NE_CHECK_ARG(kv_dtype == NE_DTYPE_BF16 || kv_dtype == NE_DTYPE_INT8,
               "kv_dtype must be bf16 or int8");
  hipStream_t s = (hipStream_t)stream;
  const int heads = num_q_heads + 2 * num_kv_heads;
  const dim3 grid((unsigned)rows * (unsigned)ceil_div(heads, 4)), block(256);
#define NE_QKR_ARGS                                                                              \
  (const uint16_t*)qkv, num_q_heads, num_kv_heads, (const uint16_t*)q_norm_weight,              \
      (const uint16_t*)k_norm_weight, eps, positions, (const uint16_t*)rope_cos_sin,           \
      rope_positions, slot_mapping, k_cache, v_cache,                                          \
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
