// QK-norm + RoPE + KV-cache write of one 128-wide head vector, shared by the row
// kernel (rowwise.hip) and the QKV GEMM's fused epilogue (gemm.hip), so that both
// produce the same bits.  Restates, per head of one token row,
// ne/models/qwen3.py:100-104 (q_norm / k_norm RMSNorm, then rotary embedding with
// the reference's cos/sin tables, qwen3.py:47-57) and
// ne/models/attention_context.py:42-54 (write_to_cache, with quantize_vectors of
// ne/models/int8_quantization.py:30-34 for an int8 cache).
//
// The vector is held by one wave: lane l has elements l and l + 64 (a, b).
#pragma once

#include "ne_common.hpp"

namespace ne {

// Where the head vectors of a QKV row go and what they need.
struct QkvRopeArgs {
  int hq, hkv;                   // query and key/value heads
  const uint16_t* q_norm_w;      // [128] bf16
  const uint16_t* k_norm_w;      // [128] bf16
  float eps;
  const int32_t* positions;      // [rows]
  const uint16_t* rope;          // [rope_positions][2][64] bf16: cos, then sin
  int rope_positions;
  const int32_t* slot_mapping;   // [rows]
  void* k_cache;                 // [slots][hkv][128] int8 or bf16
  void* v_cache;
  void* k_scale;                 // [slots][hkv] (int8 cache only)
  void* v_scale;
  uint16_t* q_out;               // [rows][hq][128] bf16
  int tiles_k;                   // row tiles of the k heads (set by the launch)
};

// Sums / maxima over the wave of N independent values, every lane ending with the same
// result.  Lanes combine within quads (DPP quad permutes), then 8 and 16 lanes (DPP
// half-row and row mirrors), then 32 (ds_swizzle xor 16), and the two halves are
// added through scalar reads of lanes 0 and 32; the N chains are interleaved so that
// their latencies overlap.  Every pairing is symmetric, so all lanes compute the same
// value in the same order.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swizzle_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <bool MAX, int N>
__device__ __forceinline__ void wave_reduce_n(float (&v)[N]) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  float t[N];
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = dpp_f32<0xB1>(v[i]);  // quad_perm [1, 0, 3, 2]
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], t[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = dpp_f32<0x4E>(v[i]);  // quad_perm [2, 3, 0, 1]
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], t[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = dpp_f32<0x141>(v[i]);  // row_half_mirror
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], t[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = dpp_f32<0x140>(v[i]);  // row_mirror
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], t[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = swizzle_xor16(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], t[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(lane_f32(v[i], 0), lane_f32(v[i], 32));
}

template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
  wave_reduce_n<false, N>(v);
}

template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
  wave_reduce_n<true, N>(v);
}

// Quantise (int8 cache) or copy N 128-vectors of one head, each held as lane /
// lane+64 values; vector i goes to slot[i] when valid[i].
template <bool INT8, int SDT, int N>
__device__ __forceinline__ void write_vectors(const float (&a)[N], const float (&b)[N], int lane,
                                              const int64_t (&slot)[N], const bool (&valid)[N], int head,
                                              int num_heads, void* cache, void* scales) {
  if constexpr (INT8) {
    float s[N];
#pragma unroll
    for (int i = 0; i < N; ++i) s[i] = fmaxf(fabsf(a[i]), fabsf(b[i]));
    wave_max_n<N>(s);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      s[i] = fmaxf(s[i], 1e-8f) / 127.f;
      // x / s as x * v_rcp_f32(s): relative error < 2e-7, so < 3e-5 at |x / s| <= 127,
      // and rint of it equals rint of the correctly rounded quotient unless it lies
      // within 1e-4 of a rounding tie; a wave with such a lane takes the exact divisions
      // (a uniform branch, skipped by most waves)
      const float rcp = __builtin_amdgcn_rcpf(s[i]);
      float ta = a[i] * rcp, tb = b[i] * rcp;
      const bool near = fabsf(ta - rintf(ta)) > 0.4999f || fabsf(tb - rintf(tb)) > 0.4999f;
      if (__builtin_amdgcn_ballot_w64(near) != 0) {
        ta = a[i] / s[i];
        tb = b[i] / s[i];
      }
      const float qa = fminf(fmaxf(rintf(ta), -127.f), 127.f);
      const float qb = fminf(fmaxf(rintf(tb), -127.f), 127.f);
      if (valid[i]) {
        int8_t* c = (int8_t*)cache + (slot[i] * num_heads + head) * 128;
        c[lane] = (int8_t)(int)qa;
        c[lane + 64] = (int8_t)(int)qb;
        if (lane == 0) store_scale<SDT>(scales, slot[i] * num_heads + head, s[i]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (valid[i]) {
        uint16_t* c = (uint16_t*)cache + (slot[i] * num_heads + head) * 128;
        c[lane] = f32_to_bf16(a[i]);
        c[lane + 64] = f32_to_bf16(b[i]);
      }
    }
  }
}

// Head h (q heads, then k heads, then v heads) of N token rows row[i], values (a, b)
// as bf16-rounded floats; only rows with valid[i] are stored.  wa / wb: the head
// type's norm weights at lane, lane + 64; c16 / s16: cos / sin of each row's
// position at lane (unused for v heads).
template <bool INT8, int SDT, int N>
__device__ __forceinline__ void qk_norm_rope_kv_vectors(const QkvRopeArgs& q, const int (&row)[N],
                                                        const bool (&valid)[N], int h, int lane,
                                                        float (&a)[N], float (&b)[N],
                                                        const int64_t (&slot)[N], float wa, float wb,
                                                        const float (&c16)[N], const float (&s16)[N]) {
  if (h < q.hq + q.hkv) {
    float ss[N];
#pragma unroll
    for (int i = 0; i < N; ++i) ss[i] = a[i] * a[i] + b[i] * b[i];
    wave_sum_n<N>(ss);
    float ra[N], rb[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float inv = rsqrtf(ss[i] / 128.f + q.eps);
      const float x = bf16_round(bf16_round(a[i] * inv) * wa);
      const float y = bf16_round(bf16_round(b[i] * inv) * wb);
      ra[i] = bf16_round(bf16_round(x * c16[i]) + bf16_round(-y * s16[i]));
      rb[i] = bf16_round(bf16_round(y * c16[i]) + bf16_round(x * s16[i]));
    }
    if (h < q.hq) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        if (valid[i]) {
          uint16_t* qo = q.q_out + ((int64_t)row[i] * q.hq + h) * 128;
          qo[lane] = f32_to_bf16(ra[i]);
          qo[lane + 64] = f32_to_bf16(rb[i]);
        }
      }
    } else {
      write_vectors<INT8, SDT, N>(ra, rb, lane, slot, valid, h - q.hq, q.hkv, q.k_cache, q.k_scale);
    }
  } else {
    write_vectors<INT8, SDT, N>(a, b, lane, slot, valid, h - q.hq - q.hkv, q.hkv, q.v_cache, q.v_scale);
  }
}

// Quantise (int8 cache) or copy one 128-vector held as lane / lane+64 values.
template <bool INT8, int SDT>
__device__ __forceinline__ void write_vector(float a, float b, int lane, int64_t slot, int head,
                                             int num_heads, void* cache, void* scales) {
  const float av[1] = {a}, bv[1] = {b};
  const int64_t sv[1] = {slot};
  const bool ok[1] = {true};
  write_vectors<INT8, SDT, 1>(av, bv, lane, sv, ok, head, num_heads, cache, scales);
}

}  // namespace ne
