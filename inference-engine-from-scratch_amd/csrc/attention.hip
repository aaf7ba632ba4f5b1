// Paged multi-query verify attention for gfx950.
//
// Replaces the reference's per-layer gather + dequant + masked SDPA
// (ne/models/attention_context.py:57-109): instead of materialising a padded
// bf16 copy of every context, K/V 16-token blocks are read in place from the
// slot pool through the block table, int8 codes are dequantised in registers
// and both products run on bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Work decomposition
//   unit  = (sequence, KV head, M tile of 16 query rows).  Row r of a unit is
//           (query head h = r / q_len within the GQA group, query i = r % q_len),
//           so 2 query heads x 5 queries (k = 4) fill 10 of the 16 MFMA rows.
//   split = a range of `split_len` keys of one unit; one 256-thread work-group
//           (4 waves) per (unit, split).  The 4 waves take interleaved 32-key
//           iterations and are merged through LDS; several splits are merged
//           by whichever work-group of the unit finishes last (atomic ticket).
//   Work-group ids are mapped so that every split of a unit lands on the
//   same XCD (ids are dealt round-robin to the 8 XCDs), keeping the partials
//   of a unit in one L2.
//
// Per 32-key iteration a wave computes S^T = K . Q^T as two 16x16 tiles
// (keys x rows, 4 MFMAs each over the 128 dims) and O^T += V^T . P^T as eight
// 16x16 tiles (dims x rows).  With S^T the softmax probabilities come out of
// the first product already in the B-operand layout of the second, so no
// shuffle is needed between them.  Lane l owns query row l % 16 and key group
// g = l / 16:
//   K load : key (l % 16) of each tile, dims 32g..32g+31 (32 B int8 / 64 B bf16)
//   V load : keys 16t + 4g + i (t < 2, i < 4), dims 8(l%16)..+8 (8 B / 16 B);
//            byte/half j of each row feeds output tile j, which transposes V
//            for free (output dim of tile j, M index m is 8m + j)
//   O      : row l % 16, dims 32g..32g+31 in registers (o[j][i] = dim 32g+8i+j)
// The MFMA contraction index is permuted consistently on both operands (dim
// 32g + 8c + e for slot 8g+e of chunk c; key 16(e/4) + 4g + e%4 for slot 8g+e),
// which is legal because a dot product does not depend on summation order.
#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kHeadDim = 128;
constexpr int kRows = 16;       // MFMA M/N tile = query rows per unit
constexpr int kIterKeys = 32;   // keys per wave iteration
constexpr int kWaves = 4;       // waves per work-group
constexpr int kThreads = kWaves * kWave;
constexpr float kNegBig = -1e30f;  // finite "minus infinity" for running maxima
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTargetWorkGroups = 1024;  // ~4 per CU on 256 CUs

struct AttnParams {
  const uint16_t* q;
  int64_t q_tok_stride, q_head_stride;
  const void* k_cache;
  const void* v_cache;
  const void* k_scale;
  const void* v_scale;
  const int32_t* block_tables;
  int32_t bt_stride;
  int32_t block_size;
  const int32_t* ctx_len;
  const int32_t* q_start;
  const int32_t* q_len;
  int32_t num_kv_heads;
  int32_t group;
  int32_t mtiles;
  int32_t max_splits;
  int32_t split_len;
  int32_t units;
  float qk_scale;  // softmax_scale * log2(e)
  uint16_t* out;
  int64_t o_tok_stride, o_head_stride;
  float* part_o;       // [units][max_splits][16][128]
  float* part_ml;      // [units][max_splits][16][2]
  uint32_t* counters;  // [units]
  uint32_t* error_flag;
};

template <bool INT8>
struct IterRegs;

template <>
struct IterRegs<true> {
  u32x4 k[2][2];  // [tile][16 B]: 32 int8 dims
  u32x2 v[8];     // [key slot e]: 8 int8 dims
  float sc;       // this lane's share of the key/value scales
};

template <>
struct IterRegs<false> {
  u32x4 k[2][4];  // [tile][16 B]: 32 bf16 dims
  u32x4 v[8];     // [key slot e]: 8 bf16 dims
  float sc;
};

__device__ __forceinline__ float sbyte(uint32_t w, int k) { return (float)(int8_t)(w >> (8 * k)); }

__device__ __forceinline__ bf16x8 int8x8_to_bf16x8(uint32_t a, uint32_t b) {
  u32x4 r = {pack_bf16x2(sbyte(a, 0), sbyte(a, 1)), pack_bf16x2(sbyte(a, 2), sbyte(a, 3)),
             pack_bf16x2(sbyte(b, 0), sbyte(b, 1)), pack_bf16x2(sbyte(b, 2), sbyte(b, 3))};
  return __builtin_bit_cast(bf16x8, r);
}

template <bool INT8, int SDT>
__device__ __forceinline__ void load_iter(const AttnParams& p, const int32_t* bt_row, int head,
                                          int kb, int kend, int lane, IterRegs<INT8>& R) {
  const int r = lane & 15;
  const int g = lane >> 4;
  const int bs = p.block_size;
  const int64_t slot_stride = (int64_t)p.num_kv_heads * kHeadDim;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int tile0 = kb + 16 * t;  // wave-uniform
    if (tile0 < kend) {
      const int blk = bt_row[tile0 / bs];
      const int64_t base_slot = (int64_t)blk * bs + (tile0 % bs);
      // K: key r of the tile, dims 32g..32g+31
      const int64_t koff = (base_slot + r) * slot_stride + (int64_t)head * kHeadDim + 32 * g;
      if constexpr (INT8) {
        const u32x4* src = (const u32x4*)((const int8_t*)p.k_cache + koff);
        R.k[t][0] = src[0];
        R.k[t][1] = src[1];
      } else {
        const u32x4* src = (const u32x4*)((const uint16_t*)p.k_cache + koff);
#pragma unroll
        for (int c = 0; c < 4; ++c) R.k[t][c] = src[c];
      }
      // V: keys 4g+i of the tile, dims 8r..8r+7
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t voff =
            (base_slot + 4 * g + i) * slot_stride + (int64_t)head * kHeadDim + 8 * r;
        if constexpr (INT8) {
          R.v[4 * t + i] = *(const u32x2*)((const int8_t*)p.v_cache + voff);
        } else {
          R.v[4 * t + i] = *(const u32x4*)((const uint16_t*)p.v_cache + voff);
        }
      }
    } else {
      if constexpr (INT8) {
        R.k[t][0] = u32x4{0, 0, 0, 0};
        R.k[t][1] = u32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) R.v[4 * t + i] = u32x2{0, 0};
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) R.k[t][c] = u32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) R.v[4 * t + i] = u32x4{0, 0, 0, 0};
      }
    }
  }
  if constexpr (INT8) {
    // lanes 0..31: key scale of key kb+lane; lanes 32..63: value scale of key kb+lane-32
    const int key = kb + (lane & 31);
    float s = 0.f;
    if (key < kend) {
      const int64_t slot = (int64_t)bt_row[key / bs] * bs + key % bs;
      const int64_t si = slot * p.num_kv_heads + head;
      s = (lane < 32) ? load_scale<SDT>(p.k_scale, si) : load_scale<SDT>(p.v_scale, si);
    }
    R.sc = s;
  }
}

template <bool INT8>
__device__ __forceinline__ void compute_iter(const AttnParams& p, const IterRegs<INT8>& R,
                                             const bf16x8 (&qf)[4], float* s_sc, int kb,
                                             int kend_row, int ctx, int lane, float& m, float& l,
                                             floatx4 (&o)[8]) {
  const int g = lane >> 4;
  // ---- S^T = K . Q^T : two 16x16 tiles (keys x rows) ----
  floatx4 s[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bf16x8 a;
      if constexpr (INT8) {
        const uint32_t* w = (const uint32_t*)&R.k[t][0];
        a = int8x8_to_bf16x8(w[2 * c], w[2 * c + 1]);
      } else {
        a = __builtin_bit_cast(bf16x8, R.k[t][c]);
      }
      s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[c], s[t], 0, 0, 0);
    }
  }
  // ---- per-key scale factors ----
  floatx4 kf[2], vf[2];
  if constexpr (INT8) {
    s_sc[lane] = R.sc;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    kf[0] = *(const floatx4*)&s_sc[4 * g];
    kf[1] = *(const floatx4*)&s_sc[16 + 4 * g];
    vf[0] = *(const floatx4*)&s_sc[32 + 4 * g];
    vf[1] = *(const floatx4*)&s_sc[48 + 4 * g];
  }
  // ---- masked scores and online softmax (row = lane % 16) ----
  float sc[8];
  float mx = kNegBig;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kb + 16 * t + 4 * g + i;
      float v = s[t][i] * p.qk_scale;
      if constexpr (INT8) v *= kf[t][i];
      v = (key < kend_row) ? v : kNegBig;
      sc[4 * t + i] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(m, mx);
  const float alpha = __builtin_amdgcn_exp2f(m - m_new);
  float pr[8];
  float psum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = kb + 16 * (e >> 2) + 4 * g + (e & 3);
    pr[e] = (key < kend_row) ? __builtin_amdgcn_exp2f(sc[e] - m_new) : 0.f;
    psum += pr[e];
  }
  l = l * alpha + psum;
  if (__ballot(alpha != 1.f)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] *= alpha;
  }
  m = m_new;
  // ---- P^T as the B operand (keys x rows), value scales folded in ----
  float pv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (INT8) {
      pv[e] = pr[e] * vf[e >> 2][e & 3];
    } else {
      pv[e] = pr[e];
    }
  }
  const u32x4 pb_bits = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]),
                         pack_bf16x2(pv[4], pv[5]), pack_bf16x2(pv[6], pv[7])};
  const bf16x8 pb = __builtin_bit_cast(bf16x8, pb_bits);
  // ---- O^T += V^T . P^T : eight 16x16 tiles (dims x rows) ----
  // bf16 values past the context end may be stale bit patterns: zero them so
  // that 0 * NaN cannot leak into the product (int8 codes are always finite).
  u32x4 vz[8];
  if constexpr (!INT8) {
    const bool tail = kb + kIterKeys > ctx;  // wave-uniform
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = kb + 16 * (e >> 2) + 4 * g + (e & 3);
      vz[e] = (tail && key >= ctx) ? u32x4{0, 0, 0, 0} : R.v[e];
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    u32x4 abits;
    if constexpr (INT8) {
      const int w = j >> 2, b = j & 3;
      abits = u32x4{pack_bf16x2(sbyte(R.v[0][w], b), sbyte(R.v[1][w], b)),
                    pack_bf16x2(sbyte(R.v[2][w], b), sbyte(R.v[3][w], b)),
                    pack_bf16x2(sbyte(R.v[4][w], b), sbyte(R.v[5][w], b)),
                    pack_bf16x2(sbyte(R.v[6][w], b), sbyte(R.v[7][w], b))};
    } else {
      const int w = j >> 1;
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      abits = u32x4{__builtin_amdgcn_perm(vz[1][w], vz[0][w], sel),
                    __builtin_amdgcn_perm(vz[3][w], vz[2][w], sel),
                    __builtin_amdgcn_perm(vz[5][w], vz[4][w], sel),
                    __builtin_amdgcn_perm(vz[7][w], vz[6][w], sel)};
    }
    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, abits), pb, o[j], 0,
                                                  0, 0);
  }
}

template <bool INT8, int SDT>
__global__ __launch_bounds__(kThreads, 3) void paged_attention_kernel(AttnParams p) {
  __shared__ float s_o[kWaves][kRows][kHeadDim + 4];
  __shared__ float s_m[kWaves][kRows];
  __shared__ float s_l[kWaves][kRows];
  __shared__ float s_sc[kWaves][kWave];
  __shared__ int s_last;

  // ---- work item ----
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int jj = bid / kNumXcd;
  const int split = jj % p.max_splits;
  const int unit = (jj / p.max_splits) * kNumXcd + xcd;
  if (unit >= p.units) return;
  const int mt = unit % p.mtiles;
  const int head = (unit / p.mtiles) % p.num_kv_heads;
  const int seq = unit / (p.mtiles * p.num_kv_heads);

  const int ctx = p.ctx_len[seq];
  const int ql = p.q_len[seq];
  const int qs = p.q_start[seq];
  const int rows_total = p.group * ql;
  const int row0 = mt * kRows;
  if (row0 >= rows_total) return;
  const int rows_here = min(kRows, rows_total - row0);
  // largest query index among this tile's rows bounds the keys it can see
  const int first_i = row0 % ql;
  const int max_i = (first_i + rows_here > ql) ? ql - 1 : first_i + rows_here - 1;
  const int kend_unit = ctx - ql + max_i + 1;
  int n_splits = (kend_unit + p.split_len - 1) / p.split_len;
  if (n_splits > p.max_splits) {
    if (threadIdx.x == 0 && split == 0) atomicOr(p.error_flag, 1u);
    n_splits = p.max_splits;
  }
  if (split >= n_splits) return;
  const int kstart = split * p.split_len;
  const int kend = min(kend_unit, kstart + p.split_len);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int R = row0 + r;
  const bool row_valid = R < rows_total;
  const int h_local = row_valid ? R / ql : 0;
  const int qi = row_valid ? R % ql : 0;
  const int kend_row = row_valid ? min(kend, ctx - ql + qi + 1) : kend;

  // ---- Q rows as the B operand: dims 32g + 8c .. +8 for chunk c ----
  bf16x8 qf[4];
  if (row_valid) {
    const int64_t qoff = (int64_t)(qs + qi) * p.q_tok_stride +
                         (int64_t)(head * p.group + h_local) * p.q_head_stride + 32 * g;
    const u32x4* src = (const u32x4*)(p.q + qoff);
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[c] = __builtin_bit_cast(bf16x8, src[c]);
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[c] = __builtin_bit_cast(bf16x8, u32x4{0, 0, 0, 0});
  }

  const int32_t* bt_row = p.block_tables + (int64_t)seq * p.bt_stride;
  float m = kNegBig, l = 0.f;
  floatx4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int n_iter = (kend - kstart + kIterKeys - 1) / kIterKeys;
  for (int it = wave; it < n_iter; it += kWaves) {
    IterRegs<INT8> A;
    load_iter<INT8, SDT>(p, bt_row, head, kstart + it * kIterKeys, kend, lane, A);
    compute_iter<INT8>(p, A, qf, s_sc[wave], kstart + it * kIterKeys, kend_row, ctx, lane, m, l, o);
  }
  // full row sum over the four key groups
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);

  // ---- merge the four waves through LDS ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    floatx4 lo = {o[0][i], o[1][i], o[2][i], o[3][i]};
    floatx4 hi = {o[4][i], o[5][i], o[6][i], o[7][i]};
    *(floatx4*)&s_o[wave][r][32 * g + 8 * i] = lo;
    *(floatx4*)&s_o[wave][r][32 * g + 8 * i + 4] = hi;
  }
  if (g == 0) {
    s_m[wave][r] = m;
    s_l[wave][r] = l;
  }
  __syncthreads();

  const int crow = tid >> 4;        // row merged by this thread
  const int cd = (tid & 15) * 8;    // its 8 dims
  float M = kNegBig;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][crow]);
  float L = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float a = __builtin_amdgcn_exp2f(s_m[w][crow] - M);
    L += a * s_l[w][crow];
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[d] += a * s_o[w][crow][cd + d];
  }

  const int CR = row0 + crow;
  const bool crow_valid = CR < rows_total;
  auto store_out = [&](const float* vals, float denom) {
    if (!crow_valid) return;
    const int ch = CR / ql, ci = CR % ql;
    const int64_t ooff = (int64_t)(qs + ci) * p.o_tok_stride +
                         (int64_t)(head * p.group + ch) * p.o_head_stride + cd;
    const float inv = 1.f / denom;
    u32x4 bits = {pack_bf16x2(vals[0] * inv, vals[1] * inv), pack_bf16x2(vals[2] * inv, vals[3] * inv),
                  pack_bf16x2(vals[4] * inv, vals[5] * inv), pack_bf16x2(vals[6] * inv, vals[7] * inv)};
    *(u32x4*)(p.out + ooff) = bits;
  };

  if (n_splits == 1) {
    store_out(acc, L);
    return;
  }

  // ---- split-K: publish this work-group's partial, last arrival merges ----
  const int64_t pbase = ((int64_t)unit * p.max_splits + split) * kRows + crow;
  float* po = p.part_o + pbase * kHeadDim + cd;
  *(floatx4*)po = floatx4{acc[0], acc[1], acc[2], acc[3]};
  *(floatx4*)(po + 4) = floatx4{acc[4], acc[5], acc[6], acc[7]};
  if ((tid & 15) == 0) {
    p.part_ml[pbase * 2] = M;
    p.part_ml[pbase * 2 + 1] = L;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&p.counters[unit], 1u);
    s_last = (prev == (uint32_t)(n_splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int64_t ubase = (int64_t)unit * p.max_splits * kRows + crow;
  float MM = kNegBig;
  for (int s = 0; s < n_splits; ++s) MM = fmaxf(MM, p.part_ml[(ubase + (int64_t)s * kRows) * 2]);
  float LL = 0.f;
  float tot[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < n_splits; ++s) {
    const int64_t pi = ubase + (int64_t)s * kRows;
    const float a = __builtin_amdgcn_exp2f(p.part_ml[pi * 2] - MM);
    LL += a * p.part_ml[pi * 2 + 1];
    const float* src = p.part_o + pi * kHeadDim + cd;
    const floatx4 x0 = *(const floatx4*)src;
    const floatx4 x1 = *(const floatx4*)(src + 4);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      tot[d] += a * x0[d];
      tot[d + 4] += a * x1[d];
    }
  }
  store_out(tot, LL);
  if (tid == 0) p.counters[unit] = 0u;  // leave the ticket ready for the next call
}

struct Layout {
  int group, mtiles, units, split_len, max_splits;
  size_t part_o_off, part_ml_off, counters_off, error_off, total;
};

Layout make_layout(int num_seqs, int num_q_heads, int num_kv_heads, int max_q_len, int max_ctx,
                   int split_len) {
  Layout L{};
  L.group = num_q_heads / num_kv_heads;
  L.mtiles = ceil_div((int64_t)L.group * max_q_len, kRows);
  L.units = num_seqs * num_kv_heads * L.mtiles;
  if (split_len <= 0) {
    const int want = max(1, ceil_div(kTargetWorkGroups, max(L.units, 1)));
    split_len = ceil_div(ceil_div(max(max_ctx, 1), want), 128) * 128;
    split_len = min(max(split_len, 128), 8192);
  }
  L.split_len = split_len;
  L.max_splits = max(1, ceil_div(max(max_ctx, 1), split_len));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  // error flag at byte 0 and tickets at byte 256, so callers can inspect and
  // re-zero them without knowing the partial-sum layout that follows
  const size_t parts = (L.max_splits > 1) ? (size_t)L.units * L.max_splits * kRows : 0;
  L.error_off = take(sizeof(uint32_t));
  L.counters_off = take((size_t)max(L.units, 1) * sizeof(uint32_t));
  L.part_o_off = take(parts * kHeadDim * sizeof(float));
  L.part_ml_off = take(parts * 2 * sizeof(float));
  L.total = off;
  return L;
}

}  // namespace

}  // namespace ne

using namespace ne;

extern "C" size_t ne_paged_attention_workspace_size(int32_t num_seqs, int32_t num_q_heads,
                                                    int32_t num_kv_heads, int32_t max_q_len,
                                                    int32_t max_ctx_len, int32_t split_len) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_q_len <= 0 ||
      num_q_heads % num_kv_heads != 0)
    return 0;
  return make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len).total;
}

extern "C" int ne_paged_verify_attention(
    const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k_cache,
    const void* v_cache, const void* k_scale, const void* v_scale, int32_t kv_dtype,
    int32_t scale_dtype, const int32_t* block_tables, int32_t block_table_stride,
    int32_t block_size, const int32_t* ctx_len, const int32_t* q_start, const int32_t* q_len,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t max_q_len, int32_t max_ctx_len, float softmax_scale, void* out,
    int64_t out_token_stride, int64_t out_head_stride, int32_t split_len, void* workspace,
    size_t workspace_bytes, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_SUPPORTED(head_dim == kHeadDim, "paged attention supports head_dim 128 only (got %d)",
                     head_dim);
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
               "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads,
               num_kv_heads);
  NE_CHECK_SUPPORTED(block_size > 0 && block_size % 16 == 0,
                     "block_size must be a positive multiple of 16 (got %d)", block_size);
  NE_CHECK_ARG(kv_dtype == NE_DTYPE_BF16 || kv_dtype == NE_DTYPE_INT8,
               "kv_dtype must be bf16 or int8");
  NE_CHECK_ARG(kv_dtype != NE_DTYPE_INT8 ||
                   (scale_dtype == NE_DTYPE_BF16 || scale_dtype == NE_DTYPE_FP16 ||
                    scale_dtype == NE_DTYPE_FP32),
               "scale_dtype must be bf16, fp16 or fp32 for an int8 cache");
  NE_CHECK_ARG(q && k_cache && v_cache && block_tables && ctx_len && q_start && q_len && out,
               "null pointer argument");
  NE_CHECK_ARG(kv_dtype != NE_DTYPE_INT8 || (k_scale && v_scale), "int8 cache needs scales");
  NE_CHECK_ARG(max_q_len > 0 && max_ctx_len > 0, "max_q_len and max_ctx_len must be positive");
  NE_CHECK_ARG(split_len == 0 || (split_len > 0 && split_len % 128 == 0),
               "split_len must be 0 or a positive multiple of 128");
  NE_CHECK_ARG((q_token_stride % 8) == 0 && (q_head_stride % 8) == 0 &&
                   (out_token_stride % 8) == 0 && (out_head_stride % 8) == 0,
               "q/out strides must be multiples of 8 elements");
  NE_CHECK_ARG(((uintptr_t)q % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                   ((uintptr_t)k_cache % 16) == 0 && ((uintptr_t)v_cache % 16) == 0,
               "q, out and caches must be 16-byte aligned");

  const Layout L =
      make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len);
  NE_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total,
               "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
               L.total);

  AttnParams p{};
  p.q = (const uint16_t*)q;
  p.q_tok_stride = q_token_stride;
  p.q_head_stride = q_head_stride;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.block_size = block_size;
  p.ctx_len = ctx_len;
  p.q_start = q_start;
  p.q_len = q_len;
  p.num_kv_heads = num_kv_heads;
  p.group = L.group;
  p.mtiles = L.mtiles;
  p.max_splits = L.max_splits;
  p.split_len = L.split_len;
  p.units = L.units;
  p.qk_scale = softmax_scale * kLog2e;
  p.out = (uint16_t*)out;
  p.o_tok_stride = out_token_stride;
  p.o_head_stride = out_head_stride;
  char* ws = (char*)workspace;
  p.part_o = (float*)(ws + L.part_o_off);
  p.part_ml = (float*)(ws + L.part_ml_off);
  p.counters = (uint32_t*)(ws + L.counters_off);
  p.error_flag = (uint32_t*)(ws + L.error_off);

  const int units_padded = ceil_div(L.units, kNumXcd) * kNumXcd;
  const dim3 grid((unsigned)units_padded * (unsigned)L.max_splits);
  hipStream_t s = (hipStream_t)stream;
  if (kv_dtype == NE_DTYPE_BF16) {
    hipLaunchKernelGGL((paged_attention_kernel<false, NE_DTYPE_BF16>), grid, dim3(kThreads), 0, s,
                       p);
  } else if (scale_dtype == NE_DTYPE_BF16) {
    hipLaunchKernelGGL((paged_attention_kernel<true, NE_DTYPE_BF16>), grid, dim3(kThreads), 0, s,
                       p);
  } else if (scale_dtype == NE_DTYPE_FP16) {
    hipLaunchKernelGGL((paged_attention_kernel<true, NE_DTYPE_FP16>), grid, dim3(kThreads), 0, s,
                       p);
  } else {
    hipLaunchKernelGGL((paged_attention_kernel<true, NE_DTYPE_FP32>), grid, dim3(kThreads), 0, s,
                       p);
  }
  return check_launch("paged_attention_kernel");
}
