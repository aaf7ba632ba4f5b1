// Paged multi-query verify attention for gfx950.
//
// Replaces the reference's per-layer gather + dequant + masked SDPA
// (ne/models/attention_context.py:57-109): instead of materialising a padded
// bf16 copy of every context, K/V 16-token blocks are read in place from the
// slot pool through the block table, int8 codes are dequantised in registers
// and both products run on MFMA (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Work decomposition
//   unit  = (sequence, KV head, M tile of 16 query rows).  Row r of a unit is
//           (query head h = r / q_len within the GQA group, query i = r % q_len),
//           so 2 query heads x 5 queries (k = 4) fill 10 of the 16 MFMA rows.
//   split = a range of keys of one sequence.  One work-group serves every KV head
//           of one (sequence, M tile, split): wave w takes KV head w, and all waves
//           walk the same 16-key tiles together, so each 1 KB (int8) slot of a
//           block is fetched whole.  Units split per KV head instead read 128-byte
//           head rows scattered in time, which a load-only probe of the same pool
//           measured at 3.2 TB/s against 4.7 TB/s for whole slots.  The split's
//           block-table slots are staged in LDS once.  The DMA kernel (int8, 8 KV
//           heads, one M tile) sizes the splits from a work plan that every
//           work-group derives from the context lengths (plan_item); the register
//           kernels use fixed `split_len` splits.
//   merge = splits store fp32 partials (reference max, sum, unnormalised output;
//           real rows only) and a second kernel combines them.  No fences or
//           atomics order the work-groups: the kernel boundary does, which on an
//           8-XCD part with one L2 per XCD is far cheaper than a device-scope
//           release per work-group.
//   int8  = codes convert to fp16 exactly with one SDWA op per value and both
//           products run on fp16 MFMA (Q is bf16, exact in fp16 for |q| < 65504);
//           the key scale multiplies the scores and the value scale is folded
//           into P.  bf16 caches use bf16 MFMA directly.
//   softmax is online with a lazily moved reference max (see compute_iter).
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
#include <type_traits>

#include <mutex>

#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kHeadDim = 128;
constexpr int kRows = 16;       // MFMA M/N tile = query rows per unit
constexpr int kIterKeys = 32;   // keys per wave iteration
constexpr int kTileKeys = 16;   // keys per MFMA tile (never straddles a block)
constexpr int kMaxSplitLen = 2048;
constexpr int kMaxTiles = kMaxSplitLen / kTileKeys;
constexpr int kPlanMaxTiles = 512;  // tiles per split of the DMA kernel's plan (8192 keys)
constexpr float kNegBig = -1e30f;  // finite "minus infinity" for running maxima
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyLog2 = 8.f;        // P <= 2^8 between rescales of the output
constexpr float kLazyMaxVScale = 128.f;  // P * scale <= 2^8 * 128 stays inside fp16
constexpr int kHeadWaves = 8;           // waves per work-group, one KV head each

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
  int32_t num_seqs;
  int32_t num_kv_heads;
  int32_t group;
  int32_t mtiles;
  int32_t max_splits;
  int32_t split_len;
  int32_t units;
  float qk_scale;  // softmax_scale * log2(e)
  uint16_t* out;
  int64_t o_tok_stride, o_head_stride;
  float* part_o;       // [units][max_splits][16][128], or [plan_grid][kv heads][16][128]
  float* part_ml;      // [units][max_splits][16][2], or [plan_grid][kv heads][16][2]
  uint32_t* error_flag;
  int32_t* plan;       // DMA kernel: first work-group of each sequence, then the total
  int32_t plan_w;      // DMA kernel: tiles per split (0: derived from the total work)
  int32_t plan_whole;  // planned path: one work item per sequence (head-split kernel)
  int32_t plan_grid;   // DMA kernel: work-groups launched
  int32_t max_ctx;     // the caller's bound on ctx_len
  int32_t* plan_desc;  // precomputed plan: [plan_grid][8] work items (seq < 0: none)
  int32_t* plan_slots; // precomputed plan: [plan_grid][kPlanMaxTiles] first slot of each tile
};

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// K/V registers of one 32-key iteration (two 16-key tiles)
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
};

// int8 codes -> fp16 (exact: |code| <= 127), one SDWA convert per value, built as a
// whole MFMA operand (4 dwords) per asm block.  The compiler sees no instruction
// inside an asm block, so it cannot insert the wait states CDNA needs between a
// VALU write of a VGPR and an MFMA reading it (two): every block ends with s_nop 1,
// which gives them to whichever instruction consumes the result.
#define NE_CVT_LO(D, S, B) "v_cvt_f16_i16_sdwa " D ", sext(" S ") dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #B "\n\t"
#define NE_CVT_HI(D, S, B) "v_cvt_f16_i16_sdwa " D ", sext(" S ") dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_" #B "\n\t"

// K operand: bytes 0..3 of w0 then of w1, in order.
__device__ __forceinline__ u32x4 i8x8_f16x8(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  asm(NE_CVT_LO("%0", "%4", 0) NE_CVT_HI("%0", "%4", 1) NE_CVT_LO("%1", "%4", 2) NE_CVT_HI("%1", "%4", 3)
      NE_CVT_LO("%2", "%5", 0) NE_CVT_HI("%2", "%5", 1) NE_CVT_LO("%3", "%5", 2) NE_CVT_HI("%3", "%5", 3)
      "s_nop 1"
      : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d)
      : "v"(w0), "v"(w1));
  return u32x4{a, b, c, d};
}

// V^T operand: byte B of each of the eight key rows x[0..7], in key order.
#define NE_CVT_COLS(B)                                                                          \
  asm(NE_CVT_LO("%0", "%4", B) NE_CVT_HI("%0", "%5", B) NE_CVT_LO("%1", "%6", B)               \
          NE_CVT_HI("%1", "%7", B) NE_CVT_LO("%2", "%8", B) NE_CVT_HI("%2", "%9", B)            \
              NE_CVT_LO("%3", "%10", B) NE_CVT_HI("%3", "%11", B) "s_nop 1"                     \
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])                                      \
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]))

template <int B>
__device__ __forceinline__ u32x4 i8_cols_f16x8(const uint32_t (&x)[8]) {
  uint32_t r[4];
  if constexpr (B == 0) {
    NE_CVT_COLS(0);
  } else if constexpr (B == 1) {
    NE_CVT_COLS(1);
  } else if constexpr (B == 2) {
    NE_CVT_COLS(2);
  } else {
    NE_CVT_COLS(3);
  }
  return u32x4{r[0], r[1], r[2], r[3]};
}
#undef NE_CVT_COLS
#undef NE_CVT_LO
#undef NE_CVT_HI

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  floatx2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// Unit geometry shared by the attention and merge kernels.
struct UnitInfo {
  int seq, head, mt, ctx, ql, qs, rows_total, row0, kend_unit, n_splits;
};

__device__ __forceinline__ UnitInfo unit_info(const AttnParams& p, int unit) {
  UnitInfo u;
  u.mt = unit % p.mtiles;
  u.head = (unit / p.mtiles) % p.num_kv_heads;
  u.seq = unit / (p.mtiles * p.num_kv_heads);
  u.ctx = p.ctx_len[u.seq];
  u.ql = p.q_len[u.seq];
  u.qs = p.q_start[u.seq];
  u.rows_total = p.group * u.ql;
  u.row0 = u.mt * kRows;
  u.kend_unit = 0;
  u.n_splits = 0;
  if (u.row0 < u.rows_total) {
    const int rows_here = min(kRows, u.rows_total - u.row0);
    // the largest query index among this tile's rows bounds the keys it can see
    const int first_i = u.row0 % u.ql;
    const int max_i = (first_i + rows_here > u.ql) ? u.ql - 1 : first_i + rows_here - 1;
    u.kend_unit = u.ctx - u.ql + max_i + 1;
    u.n_splits = max(0, (u.kend_unit + p.split_len - 1) / p.split_len);
  }
  return u;
}

// Per-wave constants for the loads: lane byte offsets inside a 16-key tile.
struct LaneOffsets {
  uint32_t k;  // key r, dims 32g..
  uint32_t v;  // key 4g, dims 8r..
  uint32_t sc; // this head's scale within a slot's scales (bytes)
};

constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

// Buffer resource over `bytes` bytes at a wave-uniform address: loads take a
// 32-bit lane offset plus an SGPR offset, and anything past `bytes` reads as 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferWord3);
}

// Issues the loads of 32-key iteration `it` of the split (clamped to the last
// iteration, whose data is then loaded again but never used).  s_slot[t] is the
// slot of the first key of the split's 16-key tile t (a tile never straddles a
// block).  Every load is a per-tile buffer resource plus a 32-bit lane offset.
template <bool INT8, int SDT>
__device__ __forceinline__ void issue_iter(const AttnParams& p, const int* s_slot, int n_tiles,
                                           int n_iter, int it, int kstart, int kend, int head,
                                           const LaneOffsets& off, int lane, IterRegs<INT8>& R) {
  constexpr int kEsz = INT8 ? 1 : 2;
  const uint32_t slot_bytes = (uint32_t)p.num_kv_heads * kHeadDim * kEsz;
  const int itc = min(it, n_iter - 1);
  const int t0 = 2 * itc;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int ti = min(t0 + t, n_tiles - 1);
    const int64_t slot = __builtin_amdgcn_readfirstlane(s_slot[ti]);
    const int64_t tile_off = slot * slot_bytes + (int64_t)head * kHeadDim * kEsz;
    const __amdgpu_buffer_rsrc_t kr =
        tile_rsrc((const char*)p.k_cache + tile_off, kTileKeys * slot_bytes);
    const __amdgpu_buffer_rsrc_t vr =
        tile_rsrc((const char*)p.v_cache + tile_off, kTileKeys * slot_bytes);
    if constexpr (INT8) {
      R.k[t][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off.k, 0, 0));
      R.k[t][1] =
          __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off.k + 16, 0, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        R.v[4 * t + i] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(vr, off.v, i * slot_bytes, 0));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        R.k[t][c] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off.k + 16 * c, 0, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        R.v[4 * t + i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, off.v, i * slot_bytes, 0));
    }
  }
  if constexpr (INT8) {
    // lanes 0..31: key scale of key kb+lane; lanes 32..63: value scale of key kb+lane-32
    // The load is unconditional (a key past kend reads its tile's first slot, which
    // is in range) and masked afterwards: a load under a lane-divergent branch
    // makes the compiler wait for every load in flight, the next iteration's too.
    const int key = kstart + itc * kIterKeys + (lane & 31);
    const int ti = min(t0 + ((lane & 31) >> 4), n_tiles - 1);
    const int64_t slot = s_slot[ti] + ((key < kend) ? (lane & 15) : 0);
    const char* base = (const char*)((lane < 32) ? p.k_scale : p.v_scale);
    constexpr int kSb = (SDT == NE_DTYPE_FP32) ? 4 : 2;
    const char* src = base + slot * p.num_kv_heads * kSb + off.sc;
    float s;
    if constexpr (SDT == NE_DTYPE_BF16) {
      s = bf16_to_f32(*(const uint16_t*)src);
    } else if constexpr (SDT == NE_DTYPE_FP16) {
      s = f16_to_f32(*(const uint16_t*)src);
    } else {
      s = *(const float*)src;
    }
    R.sc = (key < kend) ? s : 0.f;
  }
}

// Q fragments of the B operand: fp16 for the int8 cache (int8 codes are exact in
// fp16, so S keeps the bf16 product's value), bf16 otherwise.
template <bool INT8>
struct QFrag;
template <>
struct QFrag<true> {
  f16x8 q[4];
};
template <>
struct QFrag<false> {
  bf16x8 q[4];
};

// One 32-key iteration: scores, online softmax, P V.
template <bool INT8>
__device__ __forceinline__ void compute_iter(const AttnParams& p, const IterRegs<INT8>& R,
                                             const QFrag<INT8>& qf, float* s_sc, int kb,
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
      if constexpr (INT8) {
        const u32x4 a = i8x8_f16x8(R.k[t][c >> 1][2 * (c & 1)], R.k[t][c >> 1][2 * (c & 1) + 1]);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), qf.q[c], s[t],
                                                      0, 0, 0);
      } else {
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, R.k[t][c]),
                                                       qf.q[c], s[t], 0, 0, 0);
      }
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
  float mx = kNegBig;  // this lane's max; the row's four lanes hold the same m
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
  // Lazy rescale: the reference max m moves only when a score passes it by more
  // than 2^kLazyLog2 (or, for int8, when a value scale is large enough that
  // P * scale could leave the fp16 range), so the common path needs neither the
  // row max across lanes nor a pass over o.
  bool grow = mx > m + kLazyLog2;
  if constexpr (INT8) {
    const float vmax = fmaxf(fmaxf(fmaxf(vf[0][0], vf[0][1]), fmaxf(vf[0][2], vf[0][3])),
                             fmaxf(fmaxf(vf[1][0], vf[1][1]), fmaxf(vf[1][2], vf[1][3])));
    grow = grow || (vmax > kLazyMaxVScale && mx > m);
  }
  if (__ballot(grow)) {
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    l *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] *= alpha;
    m = m_new;
  }
  float pr[8];
  float psum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = kb + 16 * (e >> 2) + 4 * g + (e & 3);
    pr[e] = (key < kend_row) ? __builtin_amdgcn_exp2f(sc[e] - m) : 0.f;
    psum += pr[e];
  }
  l += psum;
  // ---- O^T += V^T . P^T : eight 16x16 tiles (dims x rows) ----
  if constexpr (INT8) {
    // value scales folded into P, which is the fp16 B operand (keys x rows)
    const u32x4 pb_bits = {pack_f16x2(pr[0] * vf[0][0], pr[1] * vf[0][1]),
                           pack_f16x2(pr[2] * vf[0][2], pr[3] * vf[0][3]),
                           pack_f16x2(pr[4] * vf[1][0], pr[5] * vf[1][1]),
                           pack_f16x2(pr[6] * vf[1][2], pr[7] * vf[1][3])};
    const f16x8 pb = __builtin_bit_cast(f16x8, pb_bits);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int w = j >> 2;
      const uint32_t col[8] = {R.v[0][w], R.v[1][w], R.v[2][w], R.v[3][w],
                               R.v[4][w], R.v[5][w], R.v[6][w], R.v[7][w]};
      u32x4 abits;
      if ((j & 3) == 0) {
        abits = i8_cols_f16x8<0>(col);
      } else if ((j & 3) == 1) {
        abits = i8_cols_f16x8<1>(col);
      } else if ((j & 3) == 2) {
        abits = i8_cols_f16x8<2>(col);
      } else {
        abits = i8_cols_f16x8<3>(col);
      }
      o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, abits), pb, o[j], 0,
                                                    0, 0);
    }
  } else {
    const u32x4 pb_bits = {pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                           pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])};
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pb_bits);
    // bf16 values past the context end may be stale bit patterns: zero them so
    // that 0 * NaN cannot leak into the product (int8 codes are always finite)
    u32x4 vz[8];
    const bool tail = kb + kIterKeys > ctx;  // wave-uniform
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = kb + 16 * (e >> 2) + 4 * g + (e & 3);
      vz[e] = (tail && key >= ctx) ? u32x4{0, 0, 0, 0} : R.v[e];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int w = j >> 1;
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      const u32x4 abits = {__builtin_amdgcn_perm(vz[1][w], vz[0][w], sel),
                           __builtin_amdgcn_perm(vz[3][w], vz[2][w], sel),
                           __builtin_amdgcn_perm(vz[5][w], vz[4][w], sel),
                           __builtin_amdgcn_perm(vz[7][w], vz[6][w], sel)};
      o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, abits), pb, o[j],
                                                     0, 0, 0);
    }
  }
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Q of one row tile for the DMA kernel's int8 product: q ~= s * (256 * hi + lo) with
// s = absmax(row) / 32512, hi in [-127, 127] and lo in [-128, 127].  The scores then run
// on the int8 MFMA straight from the cache's codes (no conversion of K), and the
// two-plane code keeps 15 bits of each row: the error, at most absmax / 65024 per
// element, is far below the bf16 rounding of Q itself.
struct QFragI8 {
  u32x4 hi[2];  // chunk c: 16 codes of dims 32g + 16c + 0..15 of this lane's row
  u32x4 lo[2];
  float c;      // qk_scale * s for this lane's row (NaN when the row is not finite)
};

constexpr float kQCodeMax = 32512.f;  // 127 * 256: hi = round(code / 256) stays in int8

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Maximum of v over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lanes of a row), by
// the gfx950 row and half-wave swaps (no LDS round trip).
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(b[0], b[1]);
}

// raw: this lane's 32 bf16 dims of its row (dims 32g + 8c + 2i, +1 in raw[c][i]).
// The code of x is round(x / s) for s = absmax / 32512, taken as the low bits of
// fma(x, 1 / s, 1.5 * 2^23 + 128) (exact integer rounding below 2^22): byte 1 of those
// bits is hi = (code + 128) >> 8 and byte 0, with its top bit flipped, is the low byte
// of lo = code - 256 hi.
__device__ __forceinline__ void quantize_q_row(const u32x4 (&raw)[4], bool valid, float qk_scale,
                                               QFragI8& f) {
  uint32_t w[16];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[4 * c + i] = valid ? raw[c][i] : 0u;
  }
  // row absmax from the bf16 magnitudes (packed 16-bit maxima); a magnitude from
  // 0x7F80 up is an infinity or NaN
  u16x2 mh = {0, 0};
#pragma unroll
  for (int j = 0; j < 16; ++j)
    mh = __builtin_elementwise_max(mh, __builtin_bit_cast(u16x2, w[j] & 0x7FFF7FFFu));
  const uint32_t mag = row_max_u32(max((uint32_t)mh[0], (uint32_t)mh[1]));
  const float amax = __uint_as_float(mag << 16);
  const float s = amax * (1.f / kQCodeMax);
  const float inv = mag != 0u ? __builtin_amdgcn_rcpf(s) : 0.f;
  constexpr float kMagic = 12583040.f;  // 1.5 * 2^23 + 128
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      // dims 16c + 4d + b: bf16 pairs w[8c + 2d] (b = 0, 1) and w[8c + 2d + 1] (b = 2, 3)
      const uint32_t w0 = w[8 * c + 2 * d], w1 = w[8 * c + 2 * d + 1];
      const uint32_t g0 = __float_as_uint(__builtin_fmaf(__uint_as_float(w0 << 16), inv, kMagic));
      const uint32_t g1 = __float_as_uint(__builtin_fmaf(__uint_as_float(w0 & 0xFFFF0000u), inv, kMagic));
      const uint32_t g2 = __float_as_uint(__builtin_fmaf(__uint_as_float(w1 << 16), inv, kMagic));
      const uint32_t g3 = __float_as_uint(__builtin_fmaf(__uint_as_float(w1 & 0xFFFF0000u), inv, kMagic));
      const uint32_t p01 = __builtin_amdgcn_perm(g1, g0, 0x04000501u);  // hi0 hi1 lo0 lo1
      const uint32_t p23 = __builtin_amdgcn_perm(g3, g2, 0x04000501u);  // hi2 hi3 lo2 lo3
      f.hi[c][d] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
      f.lo[c][d] = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;
    }
  }
  f.c = mag < 0x7F80u ? qk_scale * s : __builtin_nanf("");
}

// One 32-key iteration of the DMA kernel over MT row tiles of 16 query rows:
// S^T = K . Q^T on the int8 MFMA (K codes as they sit in LDS, Q in two int8 planes),
// the lazy online softmax, and O^T += V^T . P^T on the fp16 MFMA with the value
// scales folded into P.  Each K chunk and V column block feeds every row tile.
// MASK = false: every key of the iteration is visible to every row (no causal or
// context-end masking needed).
template <int MT, bool MASK>
__device__ __forceinline__ void compute_iter_q8(const IterRegs<true>& R, const QFragI8 (&qf)[MT],
                                                float* s_sc, int kb, const int (&kend_row)[MT],
                                                int lane, float (&m)[MT], float (&l)[MT],
                                                floatx4 (&o)[MT][8]) {
  const int g = lane >> 4;
  // ---- integer scores: 256 * (K . Qhi) + K . Qlo, exact in int32 ----
  i32x4 shi[MT][2], slo[MT][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      shi[mt][t] = i32x4{0, 0, 0, 0};
      slo[mt][t] = i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const i32x4 a = __builtin_bit_cast(i32x4, R.k[t][c]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        shi[mt][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, __builtin_bit_cast(i32x4, qf[mt].hi[c]),
                                                           shi[mt][t], 0, 0, 0);
        slo[mt][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, __builtin_bit_cast(i32x4, qf[mt].lo[c]),
                                                           slo[mt][t], 0, 0, 0);
      }
    }
  }
  // ---- per-key scale factors (lanes 0..31 key scales, 32..63 value scales) ----
  s_sc[lane] = R.sc;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const floatx4 kf0 = *(const floatx4*)&s_sc[4 * g];
  const floatx4 kf1 = *(const floatx4*)&s_sc[16 + 4 * g];
  const floatx4 vf0 = *(const floatx4*)&s_sc[32 + 4 * g];
  const floatx4 vf1 = *(const floatx4*)&s_sc[48 + 4 * g];
  const float vmax = fmaxf(fmaxf(fmaxf(vf0[0], vf0[1]), fmaxf(vf0[2], vf0[3])),
                           fmaxf(fmaxf(vf1[0], vf1[1]), fmaxf(vf1[2], vf1[3])));
  // ---- scores up to the row factor c (score = c * sc), lazy online softmax, P ----
  f16x8 pb[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const float c = qf[mt].c;
    float sc[8];
    float mx = kNegBig;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int si = (shi[mt][t][i] << 8) + slo[mt][t][i];
        float v = (float)si * (t ? kf1[i] : kf0[i]);
        if constexpr (MASK) v = (kb + 16 * t + 4 * g + i < kend_row[mt]) ? v : kNegBig;
        sc[4 * t + i] = v;
        mx = fmaxf(mx, v);
      }
    }
    mx *= c;
    const bool grow = (mx > m[mt] + kLazyLog2) || (vmax > kLazyMaxVScale && mx > m[mt]);
    if (__ballot(grow)) {
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m[mt], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[mt] - m_new);
      l[mt] *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[mt][j] *= alpha;
      m[mt] = m_new;
    }
    float pr[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], c, -m[mt]));
      if constexpr (MASK) pr[e] = (kb + 16 * (e >> 2) + 4 * g + (e & 3) < kend_row[mt]) ? pr[e] : 0.f;
      psum += pr[e];
    }
    l[mt] += psum;
    const u32x4 pb_bits = {pack_f16x2(pr[0] * vf0[0], pr[1] * vf0[1]), pack_f16x2(pr[2] * vf0[2], pr[3] * vf0[3]),
                           pack_f16x2(pr[4] * vf1[0], pr[5] * vf1[1]), pack_f16x2(pr[6] * vf1[2], pr[7] * vf1[3])};
    pb[mt] = __builtin_bit_cast(f16x8, pb_bits);
  }
  // ---- O^T += V^T . P^T: eight 16x16 tiles (dims x rows) per row tile ----
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int w = j >> 2;
    const uint32_t col[8] = {R.v[0][w], R.v[1][w], R.v[2][w], R.v[3][w],
                             R.v[4][w], R.v[5][w], R.v[6][w], R.v[7][w]};
    u32x4 abits;
    if ((j & 3) == 0) {
      abits = i8_cols_f16x8<0>(col);
    } else if ((j & 3) == 1) {
      abits = i8_cols_f16x8<1>(col);
    } else if ((j & 3) == 2) {
      abits = i8_cols_f16x8<2>(col);
    } else {
      abits = i8_cols_f16x8<3>(col);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      o[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, abits), pb[mt], o[mt][j],
                                                        0, 0, 0);
  }
}

// One work-group per (sequence, M tile, split) with kHeadWaves * KG waves.  Wave
// w serves KV heads w % kHeadWaves (+ kHeadWaves, ...) and takes every KG-th
// 32-key iteration of the split; the KG partial results of a head are merged
// through LDS.  All waves walk the same 16-key tiles at about the same time, so a
// block's 1 KB (int8) slots are fetched whole rather than as 128-byte head rows
// scattered in time.  DB: double-buffer the registers, keeping the next
// iteration's loads in flight during the current one's arithmetic.
template <bool INT8, int SDT, int KG, bool DB>
__global__ __launch_bounds__(kHeadWaves * KG * kWave) void paged_attention_kernel(AttnParams p) {
  constexpr int kWaves = kHeadWaves * KG;
  constexpr int kThreads = kWaves * kWave;
  __shared__ float s_sc[INT8 ? kWaves : 1][kWave];
  __shared__ int s_slot[kMaxTiles];
  __shared__ float s_o[KG > 1 ? kHeadWaves : 1][kRows][kHeadDim + 4];
  __shared__ float s_ml[KG > 1 ? kHeadWaves : 1][kRows][2];

  // ---- work item ----
  const int bid = blockIdx.x;
  const int split = bid % p.max_splits;
  const int mt = (bid / p.max_splits) % p.mtiles;
  const int seq = bid / (p.max_splits * p.mtiles);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int head_slot = wave % kHeadWaves;
  const int kg = wave / kHeadWaves;
  // the geometry below does not depend on the head
  const UnitInfo u0 = unit_info(p, seq * p.num_kv_heads * p.mtiles + mt);
  if (u0.row0 >= u0.rows_total) return;
  int n_splits = u0.n_splits;
  if (n_splits > p.max_splits) {
    if (tid == 0 && split == 0) atomicOr(p.error_flag, 1u);
    n_splits = p.max_splits;
  }
  if (split >= n_splits) return;
  const int kstart = split * p.split_len;
  const int kend = min(u0.kend_unit, kstart + p.split_len);
  const int ql = u0.ql;

  // ---- block-table slots of this split's 16-key tiles ----
  const int32_t* bt_row = p.block_tables + (int64_t)seq * p.bt_stride;
  const int n_tiles = (kend - kstart + kTileKeys - 1) / kTileKeys;
  for (int t = tid; t < n_tiles; t += kThreads) {
    const int key0 = kstart + kTileKeys * t;
    s_slot[t] = bt_row[key0 / p.block_size] * p.block_size + key0 % p.block_size;
  }
  __syncthreads();  // s_slot ready

  const int r = lane & 15;
  const int g = lane >> 4;
  const int R = u0.row0 + r;
  const bool row_valid = R < u0.rows_total;
  const int h_local = row_valid ? R / ql : 0;
  const int qi = row_valid ? R % ql : 0;
  const int kend_row = row_valid ? min(kend, u0.ctx - ql + qi + 1) : kend;
  const int n_iter = (kend - kstart + kIterKeys - 1) / kIterKeys;
  constexpr int kEsz = INT8 ? 1 : 2;
  const int64_t slot_bytes = (int64_t)p.num_kv_heads * kHeadDim * kEsz;

  for (int pass = 0; pass * kHeadWaves < p.num_kv_heads; ++pass) {
    const int head = pass * kHeadWaves + head_slot;
    const bool active = head < p.num_kv_heads;  // wave-uniform
    float m = kNegBig, l = 0.f;
    floatx4 o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (active) {
      // ---- Q rows as the B operand: dims 32g + 8c .. +8 for chunk c ----
      QFrag<INT8> qf;
      {
        u32x4 raw[4] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
        if (row_valid) {
          const int64_t qoff = (int64_t)(u0.qs + qi) * p.q_tok_stride +
                               (int64_t)(head * p.group + h_local) * p.q_head_stride + 32 * g;
          const u32x4* src = (const u32x4*)(p.q + qoff);
#pragma unroll
          for (int c = 0; c < 4; ++c) raw[c] = src[c];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if constexpr (INT8) {
            u32x4 h;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              h[i] = pack_f16x2(bf16_to_f32((uint16_t)(raw[c][i] & 0xFFFFu)),
                                bf16_to_f32((uint16_t)(raw[c][i] >> 16)));
            qf.q[c] = __builtin_bit_cast(f16x8, h);
          } else {
            qf.q[c] = __builtin_bit_cast(bf16x8, raw[c]);
          }
        }
      }
      LaneOffsets off;
      off.k = (uint32_t)(r * slot_bytes + 32 * g * kEsz);
      off.v = (uint32_t)(4 * g * slot_bytes + 8 * r * kEsz);
      off.sc = (uint32_t)(head * (SDT == NE_DTYPE_FP32 ? 4 : 2));
      float* sc_row = s_sc[INT8 ? wave : 0];
      if constexpr (DB) {
        IterRegs<INT8> A, B;
        issue_iter<INT8, SDT>(p, s_slot, n_tiles, n_iter, kg, kstart, kend, head, off, lane, A);
        for (int it = kg; it < n_iter; it += 2 * KG) {
          issue_iter<INT8, SDT>(p, s_slot, n_tiles, n_iter, it + KG, kstart, kend, head, off, lane,
                                B);
          compute_iter<INT8>(p, A, qf, sc_row, kstart + it * kIterKeys, kend_row, u0.ctx, lane, m,
                             l, o);
          issue_iter<INT8, SDT>(p, s_slot, n_tiles, n_iter, it + 2 * KG, kstart, kend, head, off,
                                lane, A);
          if (it + KG < n_iter)
            compute_iter<INT8>(p, B, qf, sc_row, kstart + (it + KG) * kIterKeys, kend_row, u0.ctx,
                               lane, m, l, o);
        }
      } else {
        for (int it = kg; it < n_iter; it += KG) {
          IterRegs<INT8> A;
          issue_iter<INT8, SDT>(p, s_slot, n_tiles, n_iter, it, kstart, kend, head, off, lane, A);
          compute_iter<INT8>(p, A, qf, sc_row, kstart + it * kIterKeys, kend_row, u0.ctx, lane, m,
                             l, o);
        }
      }
      // full row sum and the row's reference max (lanes of a row agree on m)
      l += __shfl_xor(l, 16);
      l += __shfl_xor(l, 32);
    }
    // ---- merge the KG key groups of each head through LDS ----
    if constexpr (KG > 1) {
      if (active && kg == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          *(floatx4*)&s_o[head_slot][r][32 * g + 8 * i] = floatx4{o[0][i], o[1][i], o[2][i], o[3][i]};
          *(floatx4*)&s_o[head_slot][r][32 * g + 8 * i + 4] =
              floatx4{o[4][i], o[5][i], o[6][i], o[7][i]};
        }
        if (g == 0) {
          s_ml[head_slot][r][0] = m;
          s_ml[head_slot][r][1] = l;
        }
      }
      __syncthreads();
      if (active && kg == 0) {
        const float m1 = s_ml[head_slot][r][0];
        const float l1 = s_ml[head_slot][r][1];
        const float mm = fmaxf(m, m1);
        const float a0 = __builtin_amdgcn_exp2f(m - mm);
        const float a1 = __builtin_amdgcn_exp2f(m1 - mm);
        l = a0 * l + a1 * l1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const floatx4 lo = *(const floatx4*)&s_o[head_slot][r][32 * g + 8 * i];
          const floatx4 hi = *(const floatx4*)&s_o[head_slot][r][32 * g + 8 * i + 4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            o[j][i] = a0 * o[j][i] + a1 * lo[j];
            o[4 + j][i] = a0 * o[4 + j][i] + a1 * hi[j];
          }
        }
        m = mm;
      }
      __syncthreads();  // s_o free for the next pass
    }
    if (!active || kg != 0 || !row_valid) continue;

    // lane (r, g) holds row r, dims 32g + 8i + j in o[j][i]
    const int unit = (seq * p.num_kv_heads + head) * p.mtiles + mt;
    if (n_splits == 1) {
      uint16_t* dst = p.out + (int64_t)(u0.qs + qi) * p.o_tok_stride +
                      (int64_t)(head * p.group + h_local) * p.o_head_stride + 32 * g;
      const float inv = 1.f / l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 bits = {pack_bf16x2(o[0][i] * inv, o[1][i] * inv),
                            pack_bf16x2(o[2][i] * inv, o[3][i] * inv),
                            pack_bf16x2(o[4][i] * inv, o[5][i] * inv),
                            pack_bf16x2(o[6][i] * inv, o[7][i] * inv)};
        *(u32x4*)(dst + 8 * i) = bits;
      }
    } else {
      // several splits: publish this split's partial for the merge kernel
      const int64_t pbase = ((int64_t)unit * p.max_splits + split) * kRows + r;
      float* po = p.part_o + pbase * kHeadDim + 32 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(floatx4*)(po + 8 * i) = floatx4{o[0][i], o[1][i], o[2][i], o[3][i]};
        *(floatx4*)(po + 8 * i + 4) = floatx4{o[4][i], o[5][i], o[6][i], o[7][i]};
      }
      if (g == 0) {
        p.part_ml[pbase * 2] = m;
        p.part_ml[pbase * 2 + 1] = l;
      }
    }
  }
}

// ---- DMA-fed variant (8 KV heads; int8 cache with 2-byte scales, or bf16) ---------
// Same work item as paged_attention_kernel, but each wave (one KV head) streams its
// head's rows of every 16-key tile, plus all heads' scales of the tile, from HBM
// straight into its own LDS ring with global_load_lds: no registers hold data in
// flight, so every wave keeps kDmaRing tiles (18 KB) on the way while it computes,
// and the loop needs no block barrier.  The scores run on the int8 MFMA with the K
// codes as they sit in LDS and Q in two int8 planes (quantize_q_row); P V stays on
// the fp16 MFMA.  A bf16 cache has twice the bytes per tile (8 KB for a head's K and V
// of 16 keys, no scales), so its ring holds two tiles per wave (the next iteration's,
// 128 KB per work-group) and the scores and P V run on the bf16 MFMA.
constexpr int kDmaRing = 4;                          // 16-key tiles in flight per wave
constexpr int kRowBytes = kHeadDim;                  // one int8 head row
constexpr int kTileRows = kTileKeys * kRowBytes;     // 2 KB: one head's K (or V) rows of a tile
constexpr int kScaleBytes = kTileKeys * kHeadWaves * 2;  // 256 B: a tile's scales, all heads
constexpr int kDmaSlot = 2 * kTileRows + 2 * kScaleBytes;  // K | V | k-scales | v-scales
constexpr int kDmaPerTile = 6;                       // 2 K + 2 V (1 KB each) + 2 scale dwords
constexpr int kPlanInts = 32;                        // LDS ints of the work plan
constexpr int kMaxRowTiles = 2;                      // row tiles per KV head in one wave
constexpr int kPartRows = kRows * kMaxRowTiles;      // rows per (work-group, KV head) partial
constexpr int kPlanMaxSeqs = 2 * kHeadWaves * kWave;  // two sequences per thread

constexpr int kBfRowBytes = kHeadDim * 2;                // one bf16 head row
constexpr int kBfTileRows = kTileKeys * kBfRowBytes;      // 4 KB: one head's K (or V) rows of a tile
constexpr int kBfDmaSlot = 2 * kBfTileRows;               // K | V
constexpr int kBfDmaPerTile = 8;                          // 4 K + 4 V copies of 1 KB

// Work-group shape of the DMA kernel by KS, the waves per KV head, and the cache dtype:
// waves per work-group, KV heads per work-group, work-groups per work item, ring tiles
// per wave, the ring slot's bytes and copies, and the dynamic LDS layout (rings, slot
// list, per-wave scales, plan).
template <int KS, bool BF16 = false>
struct DmaShape {
  static constexpr int waves = kHeadWaves;
  static constexpr int heads = waves / KS;               // KV heads per work-group
  static constexpr int groups = kHeadWaves / heads;      // work-groups per work item
  static constexpr int ring = BF16 ? 2 : kDmaRing;       // tiles in flight per wave
  static constexpr int slot_bytes = BF16 ? kBfDmaSlot : kDmaSlot;
  static constexpr int per_tile = BF16 ? kBfDmaPerTile : kDmaPerTile;  // copies per tile
  // tiles a wave with more tiles than its ring issues before the first iteration; the
  // rest of the ring follows once the first two have landed, which keeps the launch's
  // opening burst of copies (and the queueing delay every wave's first tiles see behind
  // it) at half the ring.  A wave with at most `ring` tiles issues them all at once.
  static constexpr int first = 2;
  static constexpr int slot_off = waves * ring * slot_bytes;
  static constexpr int sc_off = slot_off + kPlanMaxTiles * 4;
  static constexpr int plan_off = sc_off + waves * kWave * 4;
  static constexpr int lds = plan_off + kPlanInts * 4;
  static_assert(waves % KS == 0 && kHeadWaves % heads == 0, "whole heads per work-group");
  static_assert(lds <= 160 * 1024, "LDS of one CU");
};
constexpr int kPlanMinTiles = 16;                     // contexts up to 256 keys are never split
constexpr int kPlanFloorTiles = 8;                    // no split shorter than 128 keys
constexpr int kPlanCUs = 256;                         // work-groups the plan aims to fill
constexpr int kWholeMaxTiles = 64;                    // longest context of a whole-sequence plan

// Waves per KV head (4 or 2) when the precomputed plan gives every sequence one
// whole work item, served by that many work-groups (one per CU at most): no split
// partials and no merge kernel.  0 when the split plan serves the shape better.
int whole_plan_ks(int num_seqs, int max_ctx, int split_len, int mtiles) {
  if (split_len != 0 || mtiles != 1 || (max_ctx + kTileKeys - 1) / kTileKeys > kWholeMaxTiles) return 0;
  if (num_seqs * 4 <= kPlanCUs) return 4;
  if (num_seqs * 2 <= kPlanCUs) return 2;
  return 0;
}

// Work plan of the DMA kernel.  Sequence b has tiles_b = ceil(ctx_b / 16) 16-key
// tiles and gets n_b = ceil(tiles_b / W) splits of near-equal length (split s
// covers tiles [tiles_b s / n_b, tiles_b (s+1) / n_b)).  W is p.plan_w when the
// caller fixed the split length; else 16 when every context fits in 16 tiles (one
// split per sequence, so no partials and no merge kernel); else
// max(8, ceil(T / (G - B))) for T = sum_b tiles_b, G = p.plan_grid work-groups and
// B sequences -- splitting is paid for already, so W only balances the longest
// split against the mean.  Both keep sum_b n_b <= G:
// the longest sequence is spread over as many work-groups as its share of T asks
// for instead of one per fixed-length split, and no CU waits for a second round
// of work-groups.  Work-group w serves split w - N_b of the sequence with
// N_b <= w < N_{b+1} (N = exclusive prefix sum of n).  Every work-group derives
// the same plan from ctx_len; work-group 0 also stores N (and N_B) for the merge.
struct PlanItem {
  int seq, split, n_splits, tiles, ctx, ql, qs;
  int j0, j1;  // the split's tiles [j0, j1) (precomputed plan only)
};

// R / d for 0 <= R < 64 and 1 <= d <= 64 without an integer division: (R + 0.5) / d
// lies at least 0.5 / d from an integer, far beyond the float reciprocal's error.
__device__ __forceinline__ int small_div(int R, int d) {
  return (int)(((float)R + 0.5f) * __builtin_amdgcn_rcpf((float)d));
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) v += __shfl_xor(v, d);
  return v;
}

// The sequences' share of the plan held by thread t: sequences 2t and 2t+1.
struct PlanScan {
  int ctx[2], ql[2], qs[2], tiles[2], n[2], first[2];  // first = N_b
  int total;                                           // sum_b n_b
};

// Called by all threads of the work-group (two barriers).
__device__ PlanScan plan_scan(const AttnParams& p, int* s_plan) {
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int B = p.num_seqs;
  PlanScan ps;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = 2 * tid + k;
    const bool ok = i < B;
    ps.ctx[k] = ok ? p.ctx_len[i] : 0;
    ps.ql[k] = ok ? p.q_len[i] : 0;
    ps.qs[k] = ok ? p.q_start[i] : 0;
  }
  // a context beyond the caller's bound is flagged and clipped to it, so that no
  // block-table entry past max_ctx is read
  if (blockIdx.x == 0 && (ps.ctx[0] > p.max_ctx || ps.ctx[1] > p.max_ctx)) atomicOr(p.error_flag, 1u);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    ps.ctx[k] = min(ps.ctx[k], p.max_ctx);
    ps.tiles[k] = (ps.ql[k] > 0 && ps.ctx[k] > 0) ? (ps.ctx[k] + kTileKeys - 1) / kTileKeys : 0;
  }
  const int tsum = wave_sum(ps.tiles[0] + ps.tiles[1]);
  if (lane == 0) s_plan[wave] = tsum;
  __syncthreads();
  int T = 0;
#pragma unroll
  for (int w = 0; w < kHeadWaves; ++w) T += s_plan[w];
  const int G = p.plan_grid;
  int W = p.plan_w;
  const int max_tiles = (p.max_ctx + kTileKeys - 1) / kTileKeys;
  if (W <= 0) {
    if (p.plan_whole)
      W = max(max_tiles, 1);  // every sequence in one item
    else
      W = max_tiles <= kPlanMinTiles ? kPlanMinTiles : max(kPlanFloorTiles, (T + (G - B) - 1) / (G - B));
  }
  if (W > kPlanMaxTiles) {
    if (tid == 0 && blockIdx.x == 0) atomicOr(p.error_flag, 1u);
    W = kPlanMaxTiles;
  }
  ps.n[0] = (ps.tiles[0] + W - 1) / W;
  ps.n[1] = (ps.tiles[1] + W - 1) / W;
  const int c = ps.n[0] + ps.n[1];
  int incl = c;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  if (lane == kWave - 1) s_plan[8 + wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kHeadWaves; ++w) {
    const int x = s_plan[8 + w];
    base += (w < wave) ? x : 0;
    total += x;
  }
  ps.first[0] = base + incl - c;
  ps.first[1] = ps.first[0] + ps.n[0];
  ps.total = total;
  if (blockIdx.x == 0) {
    if (2 * tid < B) p.plan[2 * tid] = ps.first[0];
    if (2 * tid + 1 < B) p.plan[2 * tid + 1] = ps.first[1];
    if (tid == 0) p.plan[B] = total;
  }
  if (total > G && tid == 0 && blockIdx.x == 0) atomicOr(p.error_flag, 1u);
  return ps;
}

// Called by all threads of the work-group; false when the work-group has no work.
__device__ bool plan_item(const AttnParams& p, int* s_plan, PlanItem& item) {
  const int tid = threadIdx.x;
  if (tid == 0) s_plan[16] = -1;  // ordered before the owner's write by plan_scan's barriers
  const PlanScan ps = plan_scan(p, s_plan);
  const int w = blockIdx.x;
  const int k = (w >= ps.first[0] && w < ps.first[1]) ? 0
                : ((w >= ps.first[1] && w < ps.first[1] + ps.n[1]) ? 1 : -1);
  if (k >= 0) {
    s_plan[16] = 2 * tid + k;
    s_plan[17] = w - (k ? ps.first[1] : ps.first[0]);
    s_plan[18] = k ? ps.n[1] : ps.n[0];
    s_plan[19] = k ? ps.tiles[1] : ps.tiles[0];
    s_plan[20] = k ? ps.ctx[1] : ps.ctx[0];
    s_plan[21] = k ? ps.ql[1] : ps.ql[0];
    s_plan[22] = k ? ps.qs[1] : ps.qs[0];
  }
  __syncthreads();
  item.seq = s_plan[16];
  if (item.seq < 0) return false;
  item.split = s_plan[17];
  item.n_splits = s_plan[18];
  item.tiles = s_plan[19];
  item.ctx = s_plan[20];
  item.ql = s_plan[21];
  item.qs = s_plan[22];
  return true;
}

// Precomputed plan (one launch per step, shared by every layer's attention call):
// work-group b of the plan kernel serves sequence b, writing the work items of its
// splits and the slot of every 16-key tile, in the layout the planned attention
// kernel reads.  Work-group 0 also marks the unused items of the grid.
constexpr int kDescInts = 8;

__global__ __launch_bounds__(kHeadWaves * kWave) void attention_plan_kernel(AttnParams p) {
  __shared__ int s_plan[kPlanInts];
  __shared__ int s_seq[8];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  // tile j = tid's block-table entry is requested before the scan, for a tile that
  // starts below max_ctx and an entry inside the row's stride (a table narrower than
  // max_ctx needs is not read past its rows); it is used only when tid < tiles, and
  // every such tile passes both bounds
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int first_entry = tid * kTileKeys / p.block_size;
  const int first_block = tid * kTileKeys < p.max_ctx && first_entry < p.bt_stride ? bt_row[first_entry] : 0;
  const PlanScan ps = plan_scan(p, s_plan);
  if (2 * tid == b || 2 * tid + 1 == b) {
    const int k = (2 * tid == b) ? 0 : 1;
    s_seq[0] = k ? ps.n[1] : ps.n[0];
    s_seq[1] = k ? ps.first[1] : ps.first[0];
    s_seq[2] = k ? ps.tiles[1] : ps.tiles[0];
    s_seq[3] = k ? ps.ctx[1] : ps.ctx[0];
    s_seq[4] = k ? ps.ql[1] : ps.ql[0];
    s_seq[5] = k ? ps.qs[1] : ps.qs[0];
  }
  if (b == 0) {  // items past the plan's total have no work
    for (int w = ps.total + tid; w < p.plan_grid; w += kHeadWaves * kWave) p.plan_desc[(int64_t)w * kDescInts] = -1;
  }
  __syncthreads();
  const int n = s_seq[0], first = s_seq[1], tiles = s_seq[2];
  for (int s = tid; s < n; s += kHeadWaves * kWave) {
    const int w = first + s;
    if (w >= p.plan_grid) break;  // flagged by plan_scan; the item is dropped
    int32_t* d = p.plan_desc + (int64_t)w * kDescInts;
    d[0] = b;
    d[1] = s;
    d[2] = n;
    d[3] = (int)((int64_t)tiles * s / n);  // the split's tiles [d[3], d[7])
    d[4] = s_seq[3];
    d[5] = s_seq[4];
    d[6] = s_seq[5];
    d[7] = (int)((int64_t)tiles * (s + 1) / n);
  }
  for (int j = tid; j < tiles; j += kHeadWaves * kWave) {
    // split s holds tiles [tiles s / n, tiles (s + 1) / n); tile j is in the last split
    // whose start is <= j
    const int s = (int)(((int64_t)(j + 1) * n - 1) / tiles);
    const int w = first + s;
    if (w >= p.plan_grid) continue;
    const int t = j - (int)((int64_t)tiles * s / n);
    const int key0 = j * kTileKeys;
    const int block = j == tid ? first_block : bt_row[key0 / p.block_size];
    p.plan_slots[(int64_t)w * kPlanMaxTiles + t] = block * p.block_size + key0 % p.block_size;
  }
}

__device__ __forceinline__ void lds_dma(const void* src, void* lds, int bytes) {
  if (bytes == 16) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
  } else {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
  }
}

// s_waitcnt with only vmcnt (N) or only lgkmcnt (0) constrained (gfx9 encoding)
template <int N>
__device__ __forceinline__ void dma_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void dma_wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// s_waitcnt vmcnt(PER * n) for a wave-uniform n in [0, MAXN]: wait until at most the
// copies of the n tiles issued last are still in flight
template <int PER, int MAXN>
__device__ __forceinline__ void dma_wait_tiles(int n) {
  if constexpr (MAXN <= 0) {
    dma_wait_vmcnt<0>();
  } else {
    if (n >= MAXN) {
      dma_wait_vmcnt<PER * MAXN>();
    } else {
      dma_wait_tiles<PER, MAXN - 1>(n);
    }
  }
}

// The copy schedule of a wave's ring of R tiles over its n tiles: a wave with at most R
// tiles requests them all before its first iteration (one round trip); a longer one
// requests its first F, and the rest of the ring once those have landed.  Iteration it
// consumes tiles 2 it and 2 it + 1 and then requests tiles 2 it + R and 2 it + 1 + R.  No
// tile past the wave's last is copied: the odd tile a last iteration lacks is masked
// there (its keys lie at or past the end), so its ring slot is never used.
template <int R, int F>
struct DmaSchedule {
  __device__ __forceinline__ static int first(int n) { return n <= R ? n : F; }
  // tiles still in flight behind tiles 2 it, 2 it + 1 when iteration it starts
  __device__ __forceinline__ static int behind(int it, int n) {
    return it == 0 ? max(first(n) - 2, 0) : max(min(n - 2 * it - 2, R - 2), 0);
  }
};

// Per-lane byte offsets of a tile copy: K/V rows land as [16 keys][128 B] with 16-byte
// chunk c of key k stored at chunk position c ^ (k & 7), which makes the fragment reads
// conflict-free.  The offsets are 32-bit and the tile's base is wave-uniform, so every
// copy is a scalar base plus a fixed lane offset (no 64-bit address arithmetic).
struct DmaLane {
  uint32_t kv[2];  // copy j: key 8j + lane / 8, chunk (lane % 8) ^ (key % 8)
  uint32_t sc;     // the lane's dword of a tile's 256 scale bytes
};

__device__ __forceinline__ DmaLane dma_lane(int lane) {
  constexpr uint32_t slot_bytes = kHeadWaves * kRowBytes;
  DmaLane d;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int key = 8 * j + (lane >> 3);
    const int chunk = (lane & 7) ^ (key & 7);
    d.kv[j] = (uint32_t)key * slot_bytes + (uint32_t)chunk * 16u;
  }
  d.sc = (uint32_t)lane * 4u;
  return d;
}

// Copy tile `t` (clamped to the split's last tile) of head `head` into ring slot `dst`.
__device__ __forceinline__ void dma_tile(const AttnParams& p, const int* s_slot, int n_tiles, int t,
                                         int head, const DmaLane& dl, char* dst) {
  const int ti = min(t, n_tiles - 1);
  const int64_t slot0 = __builtin_amdgcn_readfirstlane(s_slot[ti]);
  const int64_t slot_bytes = (int64_t)kHeadWaves * kRowBytes;
  const char* kbase = (const char*)p.k_cache + slot0 * slot_bytes + head * kRowBytes;
  const char* vbase = (const char*)p.v_cache + slot0 * slot_bytes + head * kRowBytes;
  // the offsets pass through an empty asm so that each address is formed here from the
  // 32-bit value (scalar base + lane offset) rather than from a hoisted 64-bit copy
  uint32_t kv0 = dl.kv[0], kv1 = dl.kv[1], sc = dl.sc;
  __asm__("" : "+v"(kv0), "+v"(kv1), "+v"(sc));
  lds_dma(kbase + kv0, dst, 16);
  lds_dma(vbase + kv0, dst + kTileRows, 16);
  lds_dma(kbase + kv1, dst + 1024, 16);
  lds_dma(vbase + kv1, dst + kTileRows + 1024, 16);
  // scales [slot][8 heads] of 2 bytes: the tile's 16 slots are 256 contiguous bytes
  lds_dma((const char*)p.k_scale + slot0 * (kHeadWaves * 2) + sc, dst + 2 * kTileRows, 4);
  lds_dma((const char*)p.v_scale + slot0 * (kHeadWaves * 2) + sc, dst + 2 * kTileRows + kScaleBytes, 4);
}

// Registers of one 32-key iteration from two ring slots (the layout load_iter gives).
// MASK = false: every key of the iteration is below kend, so no scale is zeroed.
template <int SDT, bool MASK>
__device__ __forceinline__ void lds_iter(const char* slot_a, const char* slot_b, int kb, int kend,
                                         int head, int lane, IterRegs<true>& R) {
  const int r = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const char* sl = t ? slot_b : slot_a;
    R.k[t][0] = *(const u32x4*)(sl + r * kRowBytes + (((2 * g) ^ (r & 7)) * 16));
    R.k[t][1] = *(const u32x4*)(sl + r * kRowBytes + (((2 * g + 1) ^ (r & 7)) * 16));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 4 * g + i;
      R.v[4 * t + i] = *(const u32x2*)(sl + kTileRows + key * kRowBytes +
                                       (((r >> 1) ^ (key & 7)) * 16) + (r & 1) * 8);
    }
  }
  // lanes 0..31: key scale of key kb+lane; lanes 32..63: value scale of key kb+lane-32
  const int kk = lane & 31;
  const char* sl = (kk >> 4) ? slot_b : slot_a;
  const uint16_t raw = *(const uint16_t*)(sl + 2 * kTileRows + (lane >> 5) * kScaleBytes +
                                          (kk & 15) * (kHeadWaves * 2) + head * 2);
  const float s = (SDT == NE_DTYPE_BF16) ? bf16_to_f32(raw) : f16_to_f32(raw);
  R.sc = (!MASK || kb + kk < kend) ? s : 0.f;
}

// bf16 cache: copy j of a head's K (or V) tile brings keys 4j .. 4j + 3, 256 B each,
// with 16-byte chunk c of key k stored at chunk position c ^ k (k < 16), which makes the
// fragment reads below conflict-free.  Offsets are 32-bit from a wave-uniform base, as
// for the int8 tiles.
struct DmaLaneBf {
  uint32_t kv[4];  // copy j: key 4j + lane / 16, chunk (lane % 16) ^ key
};

__device__ __forceinline__ DmaLaneBf dma_lane_bf(int lane) {
  constexpr uint32_t slot_bytes = kHeadWaves * kBfRowBytes;
  DmaLaneBf d;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int key = 4 * j + (lane >> 4);
    const int chunk = (lane & 15) ^ key;
    d.kv[j] = (uint32_t)key * slot_bytes + (uint32_t)chunk * 16u;
  }
  return d;
}

// Copy tile `t` (clamped to the split's last tile) of head `head` of a bf16 cache into
// ring slot `dst`: K rows, then V rows, 4 KB each.
__device__ __forceinline__ void dma_tile_bf(const AttnParams& p, const int* s_slot, int n_tiles, int t, int head,
                                            const DmaLaneBf& dl, char* dst) {
  const int ti = min(t, n_tiles - 1);
  const int64_t slot0 = __builtin_amdgcn_readfirstlane(s_slot[ti]);
  const int64_t slot_bytes = (int64_t)kHeadWaves * kBfRowBytes;
  const char* kbase = (const char*)p.k_cache + slot0 * slot_bytes + head * kBfRowBytes;
  const char* vbase = (const char*)p.v_cache + slot0 * slot_bytes + head * kBfRowBytes;
  uint32_t o0 = dl.kv[0], o1 = dl.kv[1], o2 = dl.kv[2], o3 = dl.kv[3];
  __asm__("" : "+v"(o0), "+v"(o1), "+v"(o2), "+v"(o3));
  lds_dma(kbase + o0, dst, 16);
  lds_dma(vbase + o0, dst + kBfTileRows, 16);
  lds_dma(kbase + o1, dst + 1024, 16);
  lds_dma(vbase + o1, dst + kBfTileRows + 1024, 16);
  lds_dma(kbase + o2, dst + 2048, 16);
  lds_dma(vbase + o2, dst + kBfTileRows + 2048, 16);
  lds_dma(kbase + o3, dst + 3072, 16);
  lds_dma(vbase + o3, dst + kBfTileRows + 3072, 16);
}

// Registers of one 32-key iteration of a bf16 cache from two ring slots: k[t][c] holds
// dims 32 g + 8 c .. + 8 of key r (the layout of the Q fragments), v[4 t + i] dims
// 8 r .. + 8 of key 16 t + 4 g + i (the layout compute_iter_bf transposes for P V).
__device__ __forceinline__ void lds_iter_bf(const char* slot_a, const char* slot_b, int lane,
                                            IterRegs<false>& R) {
  const int r = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const char* sl = t ? slot_b : slot_a;
#pragma unroll
    for (int c = 0; c < 4; ++c) R.k[t][c] = *(const u32x4*)(sl + r * kBfRowBytes + (((4 * g + c) ^ r) * 16));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 4 * g + i;
      R.v[4 * t + i] = *(const u32x4*)(sl + kBfTileRows + key * kBfRowBytes + ((r ^ key) * 16));
    }
  }
}

// One 32-key iteration of a bf16 cache for MT row tiles: scores on the bf16 MFMA, the
// lazy online softmax, P V on the bf16 MFMA (the register kernel's arithmetic, each K
// and V operand feeding every row tile).  MASK: keys at or past a row's end are masked,
// and the V rows of keys at or past kend (where a partial or clamped tile holds other or
// stale slots) are zeroed, so that 0 * NaN cannot reach the product.
template <int MT, bool MASK>
__device__ __forceinline__ void compute_iter_bf(const IterRegs<false>& R, const QFrag<false> (&qf)[MT],
                                                float qk_scale, int kb, int kend, const int (&kend_row)[MT],
                                                int lane, float (&m)[MT], float (&l)[MT],
                                                floatx4 (&o)[MT][8]) {
  const int g = lane >> 4;
  // ---- S^T = K . Q^T: two 16x16 tiles (keys x rows) per row tile ----
  floatx4 s[MT][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) s[mt][t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8 a = __builtin_bit_cast(bf16x8, R.k[t][c]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        s[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[mt].q[c], s[mt][t], 0, 0, 0);
    }
  }
  // ---- masked scores, lazy online softmax, P (row = lane % 16) ----
  bf16x8 pb[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    float sc[8];
    float mx = kNegBig;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = s[mt][t][i] * qk_scale;
        if constexpr (MASK) v = (kb + 16 * t + 4 * g + i < kend_row[mt]) ? v : kNegBig;
        sc[4 * t + i] = v;
        mx = fmaxf(mx, v);
      }
    }
    if (__ballot(mx > m[mt] + kLazyLog2)) {
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m[mt], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[mt] - m_new);
      l[mt] *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[mt][j] *= alpha;
      m[mt] = m_new;
    }
    float pr[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pr[e] = __builtin_amdgcn_exp2f(sc[e] - m[mt]);
      if constexpr (MASK) pr[e] = (kb + 16 * (e >> 2) + 4 * g + (e & 3) < kend_row[mt]) ? pr[e] : 0.f;
      psum += pr[e];
    }
    l[mt] += psum;
    const u32x4 pb_bits = {pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]), pack_bf16x2(pr[4], pr[5]),
                           pack_bf16x2(pr[6], pr[7])};
    pb[mt] = __builtin_bit_cast(bf16x8, pb_bits);
  }
  // ---- O^T += V^T . P^T: eight 16x16 tiles (dims x rows) per row tile ----
  u32x4 vz[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = kb + 16 * (e >> 2) + 4 * g + (e & 3);
    vz[e] = (MASK && key >= kend) ? u32x4{0, 0, 0, 0} : R.v[e];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int w = j >> 1;
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    const u32x4 abits = {__builtin_amdgcn_perm(vz[1][w], vz[0][w], sel), __builtin_amdgcn_perm(vz[3][w], vz[2][w], sel),
                         __builtin_amdgcn_perm(vz[5][w], vz[4][w], sel), __builtin_amdgcn_perm(vz[7][w], vz[6][w], sel)};
    const bf16x8 a = __builtin_bit_cast(bf16x8, abits);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      o[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[mt], o[mt][j], 0, 0, 0);
  }
}

// PLANNED: the work item and the split's slots come from attention_plan_kernel's
// output instead of being derived here (one round trip instead of two).
// MT: row tiles of 16 per KV head handled by each wave (1, or 2 for up to 32 rows).
// KS: waves per KV head.  KS = 1: the 8 waves are the 8 KV heads of one work item.
// KS > 1 (planned, one row tile, items of whole sequences): KS work-groups share an
// item, each taking 8 / KS heads, and a head's KS waves take consecutive parts of the
// item's tiles, their (m, l, O) merged through LDS before the store -- so that short
// contexts fill KS times as many CUs without a merge kernel.
// BF16: a bf16 cache (SDT unused): two-tile rings, bf16 MFMA scores (compute_iter_bf).
template <int SDT, bool PLANNED, int MT, int KS = 1, bool BF16 = false>
__global__ __launch_bounds__((DmaShape<KS, BF16>::waves * kWave)) void paged_attention_dma_kernel(AttnParams p) {
  static_assert(KS == 1 || (PLANNED && MT == 1), "head split: planned, one row tile");
  using Shape = DmaShape<KS, BF16>;
  constexpr int HG = Shape::heads;  // KV heads per work-group
  constexpr int RING = Shape::ring;
  constexpr int FIRST = Shape::first;
  constexpr int kThreads = Shape::waves * kWave;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* s_slot = (int*)(smem + Shape::slot_off);
  float* s_sc_all = (float*)(smem + Shape::sc_off);
  int* s_plan = (int*)(smem + Shape::plan_off);

  // ---- work item: one split of one sequence (M tile 0); wave -> (KV head, part) ----
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int widx = (int)blockIdx.x / Shape::groups;  // work item
  const int head = ((int)blockIdx.x % Shape::groups) * HG + wave % HG;
  const int ks = wave / HG;  // this wave's part of the item's tiles
  const int lane = tid % kWave;
  PlanItem item;
  int32_t planned_slot = 0;
  if constexpr (PLANNED) {
    // The split's slot list (one dword per thread; entries past its tiles are never
    // read) and the work item (through the scalar cache) are requested together, and
    // the slot is stored to LDS only after the Q loads are issued, so that a single
    // round trip precedes the first K/V copy.  The compiler barriers keep the load
    // first and the store last.
    static_assert(kPlanMaxTiles == kThreads, "one slot per thread");
    const int32_t my_slot = p.plan_slots[(int64_t)widx * kPlanMaxTiles + tid];
    __asm__ __volatile__("" ::: "memory");
    const ConstI32* d = (const ConstI32*)(p.plan_desc + (int64_t)widx * kDescInts);
    item.seq = d[0];
    item.split = d[1];
    item.n_splits = d[2];
    item.j0 = d[3];
    item.ctx = d[4];
    item.ql = d[5];
    item.qs = d[6];
    item.j1 = d[7];
    // a work item that this metadata cannot have produced (no plan, or a stale one) is
    // flagged and skipped rather than followed
    const bool sane = item.seq < p.num_seqs && item.n_splits >= 1 && item.split >= 0 &&
                      item.split < item.n_splits && item.ctx > 0 && item.ctx <= p.max_ctx &&
                      item.j0 >= 0 && item.j0 < item.j1 && item.j1 - item.j0 <= kPlanMaxTiles &&
                      (item.j1 - 1) * kTileKeys < item.ctx && item.ql > 0 && item.qs >= 0;
    if (item.seq < 0 || !sane) {
      if (item.seq >= 0 && tid == 0) atomicOr(p.error_flag, 2u);
      return;
    }
    planned_slot = my_slot;
  } else {
    if (!plan_item(p, s_plan, item)) return;
  }
  // the item is the same for the whole work-group: keep it in scalar registers, so
  // that the loop and its waits are compiled as uniform
  item.seq = __builtin_amdgcn_readfirstlane(item.seq);
  item.split = __builtin_amdgcn_readfirstlane(item.split);
  item.n_splits = __builtin_amdgcn_readfirstlane(item.n_splits);
  item.ctx = __builtin_amdgcn_readfirstlane(item.ctx);
  item.ql = __builtin_amdgcn_readfirstlane(item.ql);
  item.qs = __builtin_amdgcn_readfirstlane(item.qs);
  const int seq = item.seq;
  const int n_splits = item.n_splits;
  int j0, j1;
  if constexpr (PLANNED) {
    j0 = item.j0;
    j1 = item.j1;
  } else {
    item.tiles = __builtin_amdgcn_readfirstlane(item.tiles);
    j0 = (int)((int64_t)item.tiles * item.split / n_splits);
    j1 = (int)((int64_t)item.tiles * (item.split + 1) / n_splits);
  }
  // this wave's tiles: part ks of KS of the item's [j0, j1)
  const int jw0 = j0 + (j1 - j0) * ks / KS;
  const int jw1 = j0 + (j1 - j0) * (ks + 1) / KS;
  const int kstart = jw0 * kTileKeys;
  const int kend = min(item.ctx, jw1 * kTileKeys);
  const int n_tiles = jw1 - jw0;
  const int ql = item.ql;
  const int rows_total = p.group * ql;
  if (rows_total > MT * kRows && tid == 0) atomicOr(p.error_flag, 1u);

  // lane (r, g) owns row mt * 16 + r of row tile mt
  const int r = lane & 15;
  const int g = lane >> 4;
  bool row_valid[MT];
  int h_local[MT], qi[MT], kend_row[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int R = mt * kRows + r;
    row_valid[mt] = R < rows_total;
    const int hq = small_div(R, ql);  // R < 32
    h_local[mt] = row_valid[mt] ? hq : 0;
    qi[mt] = row_valid[mt] ? R - hq * ql : 0;
    kend_row[mt] = row_valid[mt] ? min(kend, item.ctx - ql + qi[mt] + 1) : kend;
  }

  // Q and the split's block-table entries are fetched together; Q is converted
  // only after the ring's first copies are issued, so no wait sits between them
  // The loads are unconditional (an invalid row re-reads the sequence's first row
  // and is zeroed after): a load under a lane-divergent branch makes the compiler
  // wait for every memory operation in flight, the ring's first copies included.
  u32x4 raw[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int64_t qoff = (int64_t)(item.qs + qi[mt]) * p.q_tok_stride +
                         (int64_t)(head * p.group + h_local[mt]) * p.q_head_stride + 32 * g;
    const u32x4* src = (const u32x4*)(p.q + qoff);
#pragma unroll
    for (int c = 0; c < 4; ++c) raw[mt][c] = src[c];
  }
  if constexpr (!PLANNED) {
    const int32_t* bt_row = p.block_tables + (int64_t)seq * p.bt_stride;
    for (int t = tid; t < n_tiles; t += kThreads) {
      const int key0 = kstart + kTileKeys * t;
      s_slot[t] = bt_row[key0 / p.block_size] * p.block_size + key0 % p.block_size;
    }
  } else {
    __asm__ __volatile__("" ::: "memory");
    s_slot[tid] = planned_slot;  // waits for the slot load alone: the Q loads are younger
  }
  __syncthreads();  // s_slot ready

  constexpr int kSlot = Shape::slot_bytes;
  constexpr int kPerTile = Shape::per_tile;
  char* ring = smem + wave * (RING * kSlot);
  const int* w_slot = s_slot + (jw0 - j0);  // this wave's tiles in the item's slot list
  const DmaLane dl = dma_lane(lane);
  const DmaLaneBf dlb = dma_lane_bf(lane);
  auto copy_tile = [&](int t, char* dst) {
    if constexpr (BF16) {
      dma_tile_bf(p, w_slot, n_tiles, t, head, dlb, dst);
    } else {
      dma_tile(p, w_slot, n_tiles, t, head, dl, dst);
    }
  };
  using Sched = DmaSchedule<RING, FIRST>;
  const int n_first = Sched::first(n_tiles);
  if (n_tiles > 0) {
#pragma unroll
    for (int j = 0; j < RING; ++j)
      if (j < n_first) copy_tile(j, ring + j * kSlot);
    // Q was issued before the ring's copies: wait for it alone (the compiler's own wait
    // would also drain the copies, since it does not order them after the Q loads)
    dma_wait_tiles<kPerTile, RING>(n_first);
  } else {
    dma_wait_vmcnt<0>();  // a wave with no tiles of the item (KS > 1) only loads Q
  }
  // Q of a row tile: two int8 planes for the int8 scores, or the bf16 rows as they are
  // (an invalid row zeroed)
  using QF = std::conditional_t<BF16, QFrag<false>, QFragI8>;
  QF qf[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if constexpr (BF16) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qf[mt].q[c] = __builtin_bit_cast(bf16x8, row_valid[mt] ? raw[mt][c] : u32x4{0, 0, 0, 0});
    } else {
      quantize_q_row(raw[mt], row_valid[mt], p.qk_scale, qf[mt]);
    }
  }

  float m[MT], l[MT];
  floatx4 o[MT][8];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m[mt] = kNegBig;
    l[mt] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  float* sc_row = s_sc_all + wave * kWave;
  const int n_iter = (n_tiles + 1) / 2;
  // iterations whose 32 keys every row sees (below the context end and the causal
  // limit of the first query) need no masking
  const int kfull = min(kend, item.ctx - ql + 1);
  const int n_full = min(n_iter, max(0, (kfull - kstart) / kIterKeys));
  auto iteration = [&](int it, auto mask, auto first) {
    constexpr bool kMask = decltype(mask)::value;
    constexpr bool kFirst = decltype(first)::value;
    // this wave's DMA of tiles 2it, 2it+1 has landed once at most the tiles issued
    // after them are still in flight
    dma_wait_tiles<kPerTile, RING - 2>(Sched::behind(kFirst ? 0 : it, n_tiles));
    const char* sa = ring + ((2 * it) % RING) * kSlot;
    const char* sb = ring + ((2 * it + 1) % RING) * kSlot;
    const int kb = kstart + it * kIterKeys;
    IterRegs<!BF16> A;
    if constexpr (BF16) {
      lds_iter_bf(sa, sb, lane, A);
    } else {
      lds_iter<SDT, kMask>(sa, sb, kb, kend, head, lane, A);
    }
    // the two slots are free once their reads have returned: refill them before the
    // arithmetic, so that each copy has the next iterations to land
    dma_wait_lgkmcnt0();
    if constexpr (kFirst) {
#pragma unroll
      for (int j = FIRST; j < RING; ++j)
        if (j >= n_first && j < n_tiles) copy_tile(j, ring + j * kSlot);
    }
    if (2 * it + RING < n_tiles) copy_tile(2 * it + RING, ring + ((2 * it) % RING) * kSlot);
    if (2 * it + 1 + RING < n_tiles) copy_tile(2 * it + 1 + RING, ring + ((2 * it + 1) % RING) * kSlot);
    if constexpr (BF16) {
      compute_iter_bf<MT, kMask>(A, qf, p.qk_scale, kb, kend, kend_row, lane, m, l, o);
    } else {
      compute_iter_q8<MT, kMask>(A, qf, sc_row, kb, kend_row, lane, m, l, o);
    }
  };
  int it = 0;
  if (n_iter > 0) {
    // the first iteration also issues the ring's remaining tiles
    if (n_full > 0) {
      iteration(0, std::false_type{}, std::true_type{});
    } else {
      iteration(0, std::true_type{}, std::true_type{});
    }
    it = 1;
  }
  for (; it < n_full; ++it) iteration(it, std::false_type{}, std::false_type{});
  for (; it < n_iter; ++it) iteration(it, std::true_type{}, std::false_type{});
  dma_wait_vmcnt<0>();  // no copy may land in LDS after the wave has left

  if constexpr (KS > 1) {
    // the KS waves of a head combine their states (the rings are free once every wave
    // is past its loop): out = sum_k 2^(m_k - M) O_k / sum_k 2^(m_k - M) l_k
    float lt = l[0];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    lds_barrier();
    floatx4* s_o = (floatx4*)smem;                   // [wave][8][lane]
    float2* s_ml = (float2*)(smem + Shape::waves * 8 * kWave * 16);  // [wave][lane]
    static_assert(Shape::waves * kWave * (8 * 16 + 8) <= Shape::slot_off, "the merge fits in the rings");
#pragma unroll
    for (int j = 0; j < 8; ++j) s_o[(wave * 8 + j) * kWave + lane] = o[0][j];
    s_ml[wave * kWave + lane] = float2{m[0], lt};
    lds_barrier();
    if (ks != 0) return;
    float M = m[0];
#pragma unroll
    for (int k = 1; k < KS; ++k) M = fmaxf(M, s_ml[(k * HG + wave) * kWave + lane].x);
    const float a0 = __builtin_amdgcn_exp2f(m[0] - M);
    lt *= a0;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[0][j] *= a0;
#pragma unroll
    for (int k = 1; k < KS; ++k) {
      const int w = k * HG + wave;
      const float2 ml = s_ml[w * kWave + lane];
      const float a = __builtin_amdgcn_exp2f(ml.x - M);
      lt += a * ml.y;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[0][j] += a * s_o[(w * 8 + j) * kWave + lane];
    }
    m[0] = M;
    l[0] = lt;
  }

  // lane (r, g) holds row r of tile mt, dims 32g + 8i + j in o[mt][j][i]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    float lt = l[mt];
    if constexpr (KS == 1) {
      lt += __shfl_xor(lt, 16);
      lt += __shfl_xor(lt, 32);
    }
    if (!row_valid[mt]) continue;
    if (n_splits == 1) {
      uint16_t* dst = p.out + (int64_t)(item.qs + qi[mt]) * p.o_tok_stride +
                      (int64_t)(head * p.group + h_local[mt]) * p.o_head_stride + 32 * g;
      const float inv = 1.f / lt;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 bits = {pack_bf16x2(o[mt][0][i] * inv, o[mt][1][i] * inv),
                            pack_bf16x2(o[mt][2][i] * inv, o[mt][3][i] * inv),
                            pack_bf16x2(o[mt][4][i] * inv, o[mt][5][i] * inv),
                            pack_bf16x2(o[mt][6][i] * inv, o[mt][7][i] * inv)};
        *(u32x4*)(dst + 8 * i) = bits;
      }
    } else {
      // partial slot: this work item's index, which the plan gives the merge too
      const int64_t pbase = ((int64_t)widx * kHeadWaves + head) * kPartRows + mt * kRows + r;
      float* po = p.part_o + pbase * kHeadDim + 32 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(floatx4*)(po + 8 * i) = floatx4{o[mt][0][i], o[mt][1][i], o[mt][2][i], o[mt][3][i]};
        *(floatx4*)(po + 8 * i + 4) = floatx4{o[mt][4][i], o[mt][5][i], o[mt][6][i], o[mt][7][i]};
      }
      if (g == 0) {
        p.part_ml[pbase * 2] = m[mt];
        p.part_ml[pbase * 2 + 1] = lt;
      }
    }
  }
}

// Measurement kernel: the planned attention's K/V (and scale) traffic alone.  It takes
// the same work items from the plan, gives each wave the same tiles, and streams them
// through the same LDS ring with the same copies and waits, but computes nothing and
// stores nothing: its time is what this access pattern costs the memory system, the
// ceiling the attention kernel is measured against.  RUNS: the items are the balanced
// runs of kv_runs_plan_kernel (tiles of several sequences, no context of their own).
template <int KS, bool BF16, bool RUNS = false>
__global__ __launch_bounds__((DmaShape<KS, BF16>::waves * kWave)) void paged_kv_stream_kernel(AttnParams p) {
  using Shape = DmaShape<KS, BF16>;
  constexpr int HG = Shape::heads;
  constexpr int RING = Shape::ring;
  constexpr int FIRST = Shape::first;
  constexpr int kSlot = Shape::slot_bytes;
  constexpr int kPerTile = Shape::per_tile;
  constexpr int kThreads = Shape::waves * kWave;
  static_assert(kPlanMaxTiles == kThreads, "one slot per thread");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* s_slot = (int*)(smem + Shape::slot_off);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int widx = (int)blockIdx.x / Shape::groups;
  const int head = ((int)blockIdx.x % Shape::groups) * HG + wave % HG;
  const int ks = wave / HG;
  const int32_t my_slot = p.plan_slots[(int64_t)widx * kPlanMaxTiles + tid];
  const ConstI32* d = (const ConstI32*)(p.plan_desc + (int64_t)widx * kDescInts);
  const int seq = d[0], split = d[1], n_splits = d[2], j0 = d[3], ctx = d[4], j1 = d[7];
  const bool sane = RUNS ? (j0 == 0 && j1 > 0 && j1 <= kPlanMaxTiles)
                         : (seq < p.num_seqs && n_splits >= 1 && split >= 0 && split < n_splits && ctx > 0 &&
                            ctx <= p.max_ctx && j0 >= 0 && j0 < j1 && j1 - j0 <= kPlanMaxTiles &&
                            (j1 - 1) * kTileKeys < ctx);
  if (seq < 0 || !sane) {
    if (seq >= 0 && tid == 0) atomicOr(p.error_flag, 2u);
    return;
  }
  s_slot[tid] = my_slot;
  __syncthreads();
  const int jw0 = __builtin_amdgcn_readfirstlane(j0 + (j1 - j0) * ks / KS);
  const int jw1 = __builtin_amdgcn_readfirstlane(j0 + (j1 - j0) * (ks + 1) / KS);
  const int n_tiles = jw1 - jw0;
  if (n_tiles <= 0) return;
  char* ring = smem + wave * (RING * kSlot);
  const int* w_slot = s_slot + (jw0 - j0);
  const DmaLane dl = dma_lane(lane);
  const DmaLaneBf dlb = dma_lane_bf(lane);
  auto copy_tile = [&](int t, char* dst) {
    if constexpr (BF16) {
      dma_tile_bf(p, w_slot, n_tiles, t, head, dlb, dst);
    } else {
      dma_tile(p, w_slot, n_tiles, t, head, dl, dst);
    }
  };
  using Sched = DmaSchedule<RING, FIRST>;
  const int n_first = Sched::first(n_tiles);
#pragma unroll
  for (int j = 0; j < RING; ++j)
    if (j < n_first) copy_tile(j, ring + j * kSlot);
  const int n_iter = (n_tiles + 1) / 2;
  for (int it = 0; it < n_iter; ++it) {
    dma_wait_tiles<kPerTile, RING - 2>(Sched::behind(it, n_tiles));
    if (it == 0) {
#pragma unroll
      for (int j = FIRST; j < RING; ++j)
        if (j >= n_first && j < n_tiles) copy_tile(j, ring + j * kSlot);
    }
    if (2 * it + RING < n_tiles) copy_tile(2 * it + RING, ring + ((2 * it) % RING) * kSlot);
    if (2 * it + 1 + RING < n_tiles) copy_tile(2 * it + 1 + RING, ring + ((2 * it + 1) % RING) * kSlot);
  }
  dma_wait_vmcnt<0>();  // no copy may land in LDS after the wave has left
}

// Measurement plan of whole-slot runs: the sequences' 16-key tiles in order (sequence 0's,
// then sequence 1's, ...), T in all, cut into plan_grid runs of near-equal length that
// cross sequence boundaries; run w holds tiles [T w / G, T (w + 1) / G).  Work-group w of
// paged_kv_stream_kernel<1, BF16, true> then reads all 8 KV heads of every tile in its
// run (wave h: head h), so each 16-slot block is fetched whole by one work-group and every
// work-group moves the same bytes.  The stream of that split is what the planned call's
// own split (whole sequences, 2 KV heads per work-group) is compared against.
__global__ __launch_bounds__(kHeadWaves * kWave) void kv_runs_plan_kernel(AttnParams p) {
  __shared__ int s_first[kPlanMaxSeqs + 1];  // first tile of each sequence, then T
  __shared__ int s_wave[kHeadWaves];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int B = p.num_seqs;
  int tiles[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = 2 * tid + k;
    const int ctx = i < B ? min(p.ctx_len[i], p.max_ctx) : 0;
    tiles[k] = ctx > 0 ? (ctx + kTileKeys - 1) / kTileKeys : 0;
  }
  const int c = tiles[0] + tiles[1];
  int incl = c;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  if (lane == kWave - 1) s_wave[wave] = incl;
  __syncthreads();
  int base = 0, T = 0;
#pragma unroll
  for (int w = 0; w < kHeadWaves; ++w) {
    const int x = s_wave[w];
    base += (w < wave) ? x : 0;
    T += x;
  }
  const int f0 = base + incl - c;
  if (2 * tid < B) s_first[2 * tid] = f0;
  if (2 * tid + 1 < B) s_first[2 * tid + 1] = f0 + tiles[0];
  if (tid == 0) s_first[B] = T;
  __syncthreads();
  const int G = p.plan_grid;
  const int w = blockIdx.x;
  const int start = (int)((int64_t)T * w / G);
  int n = (int)((int64_t)T * (w + 1) / G) - start;
  if (n > kPlanMaxTiles) {  // the workspace's plan_grid keeps T / G below this
    if (tid == 0) atomicOr(p.error_flag, 1u);
    n = kPlanMaxTiles;
  }
  if (tid == 0) {
    int32_t* d = p.plan_desc + (int64_t)w * kDescInts;
    d[0] = n > 0 ? 0 : -1;
    d[1] = 0;
    d[2] = 1;
    d[3] = 0;  // the run's tiles [d[3], d[7])
    d[4] = 0;
    d[5] = 0;
    d[6] = 0;
    d[7] = n;
  }
  if (tid < n) {
    // tile g lies in the last sequence whose first tile is <= g (an empty sequence shares
    // its first tile with the next one, which then is the last such sequence)
    const int g = start + tid;
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (s_first[mid] <= g)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int key0 = (g - s_first[lo]) * kTileKeys;
    const int entry = key0 / p.block_size;
    int slot = 0;
    if (entry < p.bt_stride)
      slot = p.block_tables[(int64_t)lo * p.bt_stride + entry] * p.block_size + key0 % p.block_size;
    else
      atomicOr(p.error_flag, 1u);
    p.plan_slots[(int64_t)w * kPlanMaxTiles + tid] = slot;
  }
}

// Partials of a row requested together by the merge kernels, so that every (m, l, O) of
// a row is requested at once rather than in a dependent chain: batches of 8, or of 16 for
// a sequence of more than 8 splits.  16 covers the ~14 splits per sequence of 16
// sequences of 256-2048 keys in one pass (8 took two: that merge ran 1.1 us longer);
// for 3 splits a batch of 16 made the merge 1 us longer than one of 8.
constexpr int kMergeBatch = 8;
constexpr int kMergeBatchWide = 16;

// Merges n partial states (m, l, O) of one query row: out = sum_s 2^(m_s - M) O_s /
// sum_s 2^(m_s - M) l_s over dims cd..cd+7.  pi(s) is the row of partial s in part_ml /
// part_o; the partials of a batch of B are all requested before any is used (a slot past
// the last partial re-reads partial s0 and is ignored: loads under a condition were
// measured to lose the batching).
template <int B, typename PartIndex>
__device__ __forceinline__ void merge_partials_batched(const AttnParams& p, int n, int cd, PartIndex pi,
                                                       uint16_t* dst) {
  float MM = kNegBig, LL = 0.f;
  float tot[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n; s0 += B) {
    float ms[B], ls[B];
    floatx4 x0[B], x1[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int64_t r = pi((s0 + j < n) ? s0 + j : s0);
      const float2 ml = *(const float2*)(p.part_ml + r * 2);
      ms[j] = (s0 + j < n) ? ml.x : kNegBig;
      ls[j] = ml.y;
      const float* src = p.part_o + r * kHeadDim + cd;
      x0[j] = *(const floatx4*)src;
      x1[j] = *(const floatx4*)(src + 4);
    }
    float Mb = MM;
#pragma unroll
    for (int j = 0; j < B; ++j) Mb = fmaxf(Mb, ms[j]);
    const float rescale = __builtin_amdgcn_exp2f(MM - Mb);
    LL *= rescale;
#pragma unroll
    for (int d = 0; d < 8; ++d) tot[d] *= rescale;
    MM = Mb;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const float a = (s0 + j < n) ? __builtin_amdgcn_exp2f(ms[j] - MM) : 0.f;
      LL += a * ls[j];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        tot[d] += a * x0[j][d];
        tot[d + 4] += a * x1[j][d];
      }
    }
  }
  const float inv = 1.f / LL;
  *(u32x4*)dst = u32x4{pack_bf16x2(tot[0] * inv, tot[1] * inv), pack_bf16x2(tot[2] * inv, tot[3] * inv),
                       pack_bf16x2(tot[4] * inv, tot[5] * inv), pack_bf16x2(tot[6] * inv, tot[7] * inv)};
}

// n is the same for every thread of a row's work-group: the choice does not diverge
template <typename PartIndex>
__device__ __forceinline__ void merge_partials(const AttnParams& p, int n, int cd, PartIndex pi, uint16_t* dst) {
  if (n > kMergeBatch)
    merge_partials_batched<kMergeBatchWide>(p, n, cd, pi, dst);
  else
    merge_partials_batched<kMergeBatch>(p, n, cd, pi, dst);
}

// Combines the partials of every sequence the plan split: one work-group per
// (sequence, KV head), 16 threads per row, 8 dims per thread; partial k of the
// sequence is work-group N_b + k's.
__global__ __launch_bounds__(kPartRows * 16) void attention_plan_merge_kernel(AttnParams p) {
  const int seq = blockIdx.x / kHeadWaves;
  const int head = blockIdx.x % kHeadWaves;
  // the sequence's plan entries and rows through the scalar cache (written by earlier kernels)
  const int first = ((const ConstI32*)p.plan)[seq];
  const int last = min(((const ConstI32*)p.plan)[seq + 1], p.plan_grid);
  const int ql = ((const ConstI32*)p.q_len)[seq];
  const int qs = ((const ConstI32*)p.q_start)[seq];
  const int n_splits = last - first;
  if (n_splits <= 1) return;
  const int crow = threadIdx.x >> 4;
  const int cd = (threadIdx.x & 15) * 8;
  if (crow >= min(p.group * ql, kPartRows)) return;
  const int ch = crow / ql, ci = crow % ql;
  uint16_t* dst = p.out + (int64_t)(qs + ci) * p.o_tok_stride +
                  (int64_t)(head * p.group + ch) * p.o_head_stride + cd;
  merge_partials(p, n_splits, cd,
                 [&](int s) { return ((int64_t)(first + s) * kHeadWaves + head) * kPartRows + crow; }, dst);
}

// Combines the split partials of every unit that has more than one split (the
// fixed-split kernels' layout): one work-group per unit, 16 threads per row, 8 dims
// per thread.
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnParams p) {
  const int unit = blockIdx.x;
  const UnitInfo u = unit_info(p, unit);
  if (u.row0 >= u.rows_total) return;
  const int n_splits = min(u.n_splits, p.max_splits);
  if (n_splits <= 1) return;
  const int crow = threadIdx.x >> 4;
  const int cd = (threadIdx.x & 15) * 8;
  const int CR = u.row0 + crow;
  if (CR >= u.rows_total) return;
  const int64_t ubase = (int64_t)unit * p.max_splits * kRows + crow;
  const int ch = CR / u.ql, ci = CR % u.ql;
  uint16_t* dst = p.out + (int64_t)(u.qs + ci) * p.o_tok_stride +
                  (int64_t)(u.head * p.group + ch) * p.o_head_stride + cd;
  merge_partials(p, n_splits, cd, [&](int s) { return ubase + (int64_t)s * kRows; }, dst);
}

struct Layout {
  int group, mtiles, units, split_len, max_splits, plan_grid, plan_w;
  size_t part_o_off, part_ml_off, error_off, plan_off, desc_off, slots_off, total;
};

// Work-groups of the DMA kernel's plan: enough that W <= kPlanMaxTiles for any
// contexts up to max_ctx (G - B >= B ceil(max_ctx / 16) / kPlanMaxTiles) and that G - B
// >= B; at least one per CU.  With a fixed split length, one per split.
int plan_grid(int num_seqs, int max_ctx, int split_len) {
  const int64_t max_tiles = ((int64_t)max(max_ctx, 1) + kTileKeys - 1) / kTileKeys;
  if (split_len > 0) {
    const int64_t w = split_len / kTileKeys;
    return (int)((int64_t)num_seqs * ((max_tiles + w - 1) / w));
  }
  const int64_t need = num_seqs + ((int64_t)num_seqs * max_tiles + kPlanMaxTiles - 1) / kPlanMaxTiles;
  int64_t g = 2 * (int64_t)num_seqs;
  if (g < kPlanCUs) g = kPlanCUs;
  if (g < need) g = need;
  return (int)g;
}

// Default split: about 512 KB of K/V per work-group (256 keys of int8, 128 of bf16,
// across 8 KV heads), the best of a sweep over 128..1024 keys on the 64-sequence
// int8 and 16-sequence bf16 verify shapes; longer splits leave CUs idle, shorter
// ones spend more on partials and per-work-group setup than they gain.
int default_split_len(int kv_dtype, int max_ctx) {
  const int split_len = (kv_dtype == NE_DTYPE_INT8) ? 256 : 128;
  return min(split_len, max(128, ceil_div(max(max_ctx, 1), 128) * 128));
}

Layout make_layout(int num_seqs, int num_q_heads, int num_kv_heads, int max_q_len, int max_ctx,
                   int split_len, int kv_dtype) {
  Layout L{};
  L.group = num_q_heads / num_kv_heads;
  L.mtiles = ceil_div((int64_t)L.group * max_q_len, kRows);
  L.units = num_seqs * num_kv_heads * L.mtiles;
  const int fixed_split = split_len > 0 ? split_len : 0;  // 0: the caller left it to us
  if (split_len <= 0) split_len = default_split_len(kv_dtype, max_ctx);
  L.split_len = split_len;
  L.max_splits = max(1, ceil_div(max(max_ctx, 1), split_len));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  // error flag at byte 0, so callers can inspect and clear it without knowing the
  // partial-sum layout that follows
  // the fixed-split kernels index partials by (unit, split); the DMA kernel's plan
  // by (work-group, KV head) and needs (B + 1) plan entries.  The sizes do not depend
  // on the cache dtype (the partials take room for either dtype's default split), so
  // the plan that ne_paged_attention_plan writes sits where a planned call of either
  // dtype reads it.
  const bool plan = num_kv_heads == kHeadWaves && L.mtiles <= kMaxRowTiles;
  L.plan_grid = plan ? plan_grid(num_seqs, max_ctx, fixed_split) : 0;
  L.plan_w = fixed_split / kTileKeys;
  int splits_room = L.max_splits;
  if (fixed_split == 0) {
    for (int dt : {NE_DTYPE_INT8, NE_DTYPE_BF16})
      splits_room = max(splits_room, ceil_div(max(max_ctx, 1), default_split_len(dt, max_ctx)));
  }
  size_t parts = (splits_room > 1) ? (size_t)L.units * splits_room * kRows : 0;
  const int plan_min_w = fixed_split > 0 ? fixed_split / kTileKeys : kPlanMinTiles;
  const bool plan_splits = ceil_div((int64_t)max(max_ctx, 1), kTileKeys) > plan_min_w;
  if (plan && plan_splits) parts = max(parts, (size_t)L.plan_grid * kHeadWaves * kPartRows);
  L.error_off = take(sizeof(uint32_t));
  L.part_o_off = take(parts * kHeadDim * sizeof(float));
  L.part_ml_off = take(parts * 2 * sizeof(float));
  L.plan_off = take(plan ? ((size_t)num_seqs + 1) * sizeof(int32_t) : 0);
  L.desc_off = take(plan ? (size_t)L.plan_grid * kDescInts * sizeof(int32_t) : 0);
  L.slots_off = take(plan ? (size_t)L.plan_grid * kPlanMaxTiles * sizeof(int32_t) : 0);
  L.total = off;
  return L;
}

template <int KG, bool DB>
int launch_attention(const AttnParams& p, int kv_dtype, int scale_dtype, hipStream_t s) {
  const dim3 grid((unsigned)p.num_seqs * (unsigned)p.mtiles * (unsigned)p.max_splits);
  const dim3 block(kHeadWaves * KG * kWave);
  if (kv_dtype == NE_DTYPE_BF16) {
    hipLaunchKernelGGL((paged_attention_kernel<false, NE_DTYPE_BF16, KG, DB>), grid, block, 0, s, p);
  } else if (scale_dtype == NE_DTYPE_BF16) {
    hipLaunchKernelGGL((paged_attention_kernel<true, NE_DTYPE_BF16, KG, DB>), grid, block, 0, s, p);
  } else if (scale_dtype == NE_DTYPE_FP16) {
    hipLaunchKernelGGL((paged_attention_kernel<true, NE_DTYPE_FP16, KG, DB>), grid, block, 0, s, p);
  } else {
    hipLaunchKernelGGL((paged_attention_kernel<true, NE_DTYPE_FP32, KG, DB>), grid, block, 0, s, p);
  }
  int rc = check_launch("paged_attention_kernel");
  if (rc != NE_OK || p.max_splits == 1) return rc;
  hipLaunchKernelGGL(attention_merge_kernel, dim3((unsigned)p.units), dim3(256), 0, s, p);
  return check_launch("attention_merge_kernel");
}

// The DMA kernel serves caches with 8 KV heads: int8 with 2-byte scales, or bf16
// (BF16); it needs the attribute for more than the default dynamic LDS once per
// instantiation.
template <int SDT, bool PLANNED, int MT, int KS = 1, bool BF16 = false>
int launch_attention_dma_ks(const AttnParams& p, unsigned grid, hipStream_t s) {
  constexpr int lds = DmaShape<KS, BF16>::lds;
  static const hipError_t attr = hipFuncSetAttribute(
      (const void*)paged_attention_dma_kernel<SDT, PLANNED, MT, KS, BF16>,
      hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) {
    set_error("paged_attention_dma_kernel: cannot reserve %d bytes of LDS: %s", lds, hipGetErrorString(attr));
    return NE_ELAUNCH;
  }
  hipLaunchKernelGGL((paged_attention_dma_kernel<SDT, PLANNED, MT, KS, BF16>), dim3(grid),
                     dim3(DmaShape<KS, BF16>::waves * kWave), lds, s, p);
  return check_launch("paged_attention_dma_kernel");
}

template <int SDT, bool PLANNED, int MT, bool BF16>
int launch_attention_dma_mt(const AttnParams& p, hipStream_t s) {
  if constexpr (PLANNED && MT == 1) {
    // whole-sequence items: 4 (or 2) work-groups per sequence, each over 2 (or 4) KV
    // heads, the waves of a head over consecutive parts of its tiles
    if (p.plan_whole) {
      if (whole_plan_ks(p.num_seqs, p.max_ctx, 0, 1) == 4)
        return launch_attention_dma_ks<SDT, PLANNED, MT, 4, BF16>(p, (unsigned)p.num_seqs * DmaShape<4>::groups, s);
      return launch_attention_dma_ks<SDT, PLANNED, MT, 2, BF16>(p, (unsigned)p.num_seqs * DmaShape<2>::groups, s);
    }
  }
  // no sequence is split when every context fits in one split's minimum length
  const int min_w = p.plan_w > 0 ? p.plan_w : kPlanMinTiles;
  const bool no_splits = ceil_div(p.max_ctx, kTileKeys) <= min_w;
  const int rc = launch_attention_dma_ks<SDT, PLANNED, MT, 1, BF16>(p, (unsigned)p.plan_grid, s);
  if (rc != NE_OK || no_splits) return rc;
  hipLaunchKernelGGL(attention_plan_merge_kernel, dim3((unsigned)p.num_seqs * kHeadWaves),
                     dim3(kPartRows * 16), 0, s, p);
  return check_launch("attention_plan_merge_kernel");
}

template <int SDT, bool PLANNED, bool BF16 = false>
int launch_attention_dma(const AttnParams& p, hipStream_t s) {
  return p.mtiles == 1 ? launch_attention_dma_mt<SDT, PLANNED, 1, BF16>(p, s)
                       : launch_attention_dma_mt<SDT, PLANNED, 2, BF16>(p, s);
}

// the DMA kernel of a parameter block whose cache dtype and scales it serves
template <bool PLANNED>
int launch_attention_dma_for(const AttnParams& p, int32_t kv_dtype, int32_t scale_dtype, hipStream_t s) {
  if (kv_dtype == NE_DTYPE_BF16) return launch_attention_dma<NE_DTYPE_BF16, PLANNED, true>(p, s);
  return scale_dtype == NE_DTYPE_BF16 ? launch_attention_dma<NE_DTYPE_BF16, PLANNED>(p, s)
                                      : launch_attention_dma<NE_DTYPE_FP16, PLANNED>(p, s);
}

// whether the DMA kernel serves this call: 8 KV heads, at most two row tiles per KV
// head, at most kPlanMaxSeqs sequences, and a bf16 cache or an int8 one with 2-byte,
// 4-byte-aligned scales
bool dma_serves(int32_t kv_dtype, int32_t scale_dtype, int32_t num_kv_heads, int mtiles, int32_t num_seqs,
                const void* k_scale, const void* v_scale) {
  if (num_kv_heads != kHeadWaves || mtiles > kMaxRowTiles || num_seqs > kPlanMaxSeqs) return false;
  if (kv_dtype == NE_DTYPE_BF16) return true;
  return kv_dtype == NE_DTYPE_INT8 && (scale_dtype == NE_DTYPE_BF16 || scale_dtype == NE_DTYPE_FP16) &&
         ((uintptr_t)k_scale % 4) == 0 && ((uintptr_t)v_scale % 4) == 0;
}

// Validates the arguments and fills the kernel parameters; NE_OK or an error code.
int make_params(const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k_cache,
                const void* v_cache, const void* k_scale, const void* v_scale, int32_t kv_dtype,
                int32_t scale_dtype, const int32_t* block_tables, int32_t block_table_stride,
                int32_t block_size, const int32_t* ctx_len, const int32_t* q_start,
                const int32_t* q_len, int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                int32_t head_dim, int32_t max_q_len, int32_t max_ctx_len, float softmax_scale,
                void* out, int64_t out_token_stride, int64_t out_head_stride, int32_t split_len,
                void* workspace, size_t workspace_bytes, AttnParams& p) {
  NE_CHECK_SUPPORTED(head_dim == kHeadDim, "paged attention supports head_dim 128 only (got %d)",
                     head_dim);
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
               "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads,
               num_kv_heads);
  NE_CHECK_SUPPORTED(block_size > 0 && block_size % kTileKeys == 0,
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
  NE_CHECK_ARG(split_len == 0 || (split_len > 0 && split_len % 128 == 0 && split_len <= kMaxSplitLen),
               "split_len must be 0 or a positive multiple of 128 up to %d", kMaxSplitLen);
  NE_CHECK_ARG((q_token_stride % 8) == 0 && (q_head_stride % 8) == 0 &&
                   (out_token_stride % 8) == 0 && (out_head_stride % 8) == 0,
               "q/out strides must be multiples of 8 elements");
  NE_CHECK_ARG(((uintptr_t)q % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                   ((uintptr_t)k_cache % 16) == 0 && ((uintptr_t)v_cache % 16) == 0,
               "q, out and caches must be 16-byte aligned");
  const Layout L = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len,
                               split_len, kv_dtype);
  NE_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total,
               "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
               L.total);
  p = AttnParams{};
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
  p.num_seqs = num_seqs;
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
  p.error_flag = (uint32_t*)(ws + L.error_off);
  p.plan = (int32_t*)(ws + L.plan_off);
  p.plan_desc = (int32_t*)(ws + L.desc_off);
  p.plan_slots = (int32_t*)(ws + L.slots_off);
  p.plan_w = L.plan_w;
  p.plan_grid = L.plan_grid;
  p.plan_whole = 0;  // the planned entry point decides
  p.max_ctx = max_ctx_len;
  return NE_OK;
}

// Device scratch of the allocation-free entry point: the work plan and split partials of
// one call, in a file-scope array each GPU holds for the life of the process.  Host code
// never passes `scratch` itself (a host-side stand-in for the symbol): it passes the
// device address hipGetSymbolAddress gives for the current device.
constexpr size_t kNoAllocScratchBytes = (size_t)NE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// the current device's scratch address, looked up once per device
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("no current HIP device (%s, device %d)", hipGetErrorString(err), dev);
    return NE_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(err));
      return NE_ELAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NE_OK;
}

// the unplanned call on a prepared parameter block (shared by both unplanned entry points)
int run_unplanned(AttnParams& p, int32_t kv_dtype, int32_t scale_dtype, int32_t num_kv_heads,
                  int32_t num_seqs, const void* k_scale, const void* v_scale, hipStream_t stream) {
  // 8 KV heads, up to two M tiles, bf16 or int8 with 2-byte scales: the DMA kernel on
  // the balanced plan.  Other int8 shapes: one wave per KV head, registers
  // double-buffered (154 VGPRs); other bf16 shapes: single-buffered (double-buffered it
  // needs 244 VGPRs).  Both on fixed-length splits.
  if (dma_serves(kv_dtype, scale_dtype, num_kv_heads, p.mtiles, num_seqs, k_scale, v_scale))
    return launch_attention_dma_for<false>(p, kv_dtype, scale_dtype, stream);
  if (kv_dtype == NE_DTYPE_INT8) return launch_attention<1, true>(p, kv_dtype, scale_dtype, stream);
  return launch_attention<1, false>(p, kv_dtype, scale_dtype, stream);
}

}  // namespace

}  // namespace ne

using namespace ne;

extern "C" size_t ne_paged_attention_workspace_size(int32_t num_seqs, int32_t num_q_heads,
                                                    int32_t num_kv_heads, int32_t max_q_len,
                                                    int32_t max_ctx_len, int32_t split_len) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_q_len <= 0 ||
      num_q_heads % num_kv_heads != 0 || split_len < 0 || split_len > kMaxSplitLen)
    return 0;
  // without an explicit split the size covers either cache dtype's default split
  const size_t a = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len,
                               split_len, NE_DTYPE_INT8).total;
  const size_t b = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len,
                               split_len, NE_DTYPE_BF16).total;
  return a > b ? a : b;
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
  AttnParams p;
  const int rc = make_params(q, q_token_stride, q_head_stride, k_cache, v_cache, k_scale, v_scale,
                             kv_dtype, scale_dtype, block_tables, block_table_stride, block_size,
                             ctx_len, q_start, q_len, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             max_q_len, max_ctx_len, softmax_scale, out, out_token_stride,
                             out_head_stride, split_len, workspace, workspace_bytes, p);
  if (rc != NE_OK) return rc;
  return run_unplanned(p, kv_dtype, scale_dtype, num_kv_heads, num_seqs, k_scale, v_scale, (hipStream_t)stream);
}

extern "C" int ne_paged_verify_attention_noalloc(
    const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k_cache,
    const void* v_cache, const void* k_scale, const void* v_scale, int32_t kv_dtype,
    int32_t scale_dtype, const int32_t* block_tables, int32_t block_table_stride,
    int32_t block_size, const int32_t* ctx_len, const int32_t* q_start, const int32_t* q_len,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t max_q_len, int32_t max_ctx_len, float softmax_scale, void* out,
    int64_t out_token_stride, int64_t out_head_stride, int32_t split_len, uint32_t* error_flag,
    void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(error_flag != nullptr && ((uintptr_t)error_flag % 4) == 0,
               "error_flag must be a 4-byte aligned device word");
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && max_q_len > 0 &&
                   max_ctx_len > 0,
               "bad attention shape");
  const Layout L = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len, kv_dtype);
  if (L.total > kNoAllocScratchBytes) {
    set_error("this call needs %zu bytes of scratch; the allocation-free entry point holds at most %zu "
              "(%d sequences, max_q_len %d, max_ctx_len %d): use ne_paged_verify_attention with a workspace",
              L.total, kNoAllocScratchBytes, num_seqs, max_q_len, max_ctx_len);
    return NE_EWORKSPACE;
  }
  void* ws = nullptr;
  int rc = scratch_for_current_device(&ws);
  if (rc != NE_OK) return rc;
  AttnParams p;
  rc = make_params(q, q_token_stride, q_head_stride, k_cache, v_cache, k_scale, v_scale, kv_dtype, scale_dtype,
                   block_tables, block_table_stride, block_size, ctx_len, q_start, q_len, num_seqs, num_q_heads,
                   num_kv_heads, head_dim, max_q_len, max_ctx_len, softmax_scale, out, out_token_stride,
                   out_head_stride, split_len, ws, kNoAllocScratchBytes, p);
  if (rc != NE_OK) return rc;
  p.error_flag = error_flag;  // the caller's word, not the scratch's
  return run_unplanned(p, kv_dtype, scale_dtype, num_kv_heads, num_seqs, k_scale, v_scale, (hipStream_t)stream);
}

extern "C" int ne_paged_attention_plan(const int32_t* block_tables, int32_t block_table_stride,
                                       int32_t block_size, const int32_t* ctx_len,
                                       const int32_t* q_start, const int32_t* q_len, int32_t num_seqs,
                                       int32_t num_q_heads, int32_t num_kv_heads, int32_t max_q_len,
                                       int32_t max_ctx_len, int32_t split_len, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
               "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads,
               num_kv_heads);
  NE_CHECK_SUPPORTED(block_size > 0 && block_size % kTileKeys == 0,
                     "block_size must be a positive multiple of 16 (got %d)", block_size);
  NE_CHECK_ARG(block_tables && ctx_len && q_start && q_len, "null pointer argument");
  NE_CHECK_ARG(max_q_len > 0 && max_ctx_len > 0, "max_q_len and max_ctx_len must be positive");
  NE_CHECK_ARG(split_len == 0 || (split_len > 0 && split_len % 128 == 0 && split_len <= kMaxSplitLen),
               "split_len must be 0 or a positive multiple of 128 up to %d", kMaxSplitLen);
  const Layout L = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len,
                               split_len, NE_DTYPE_INT8);
  NE_CHECK_SUPPORTED(num_kv_heads == kHeadWaves && L.mtiles <= kMaxRowTiles && num_seqs <= kPlanMaxSeqs,
                     "a precomputed plan serves 8 KV heads, at most %d query rows per KV head "
                     "and at most %d sequences", kMaxRowTiles * kRows, kPlanMaxSeqs);
  NE_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total,
               "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
  AttnParams p{};
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.block_size = block_size;
  p.ctx_len = ctx_len;
  p.q_start = q_start;
  p.q_len = q_len;
  p.num_seqs = num_seqs;
  p.num_kv_heads = num_kv_heads;
  p.group = L.group;
  p.mtiles = L.mtiles;
  p.max_ctx = max_ctx_len;
  p.plan_w = L.plan_w;
  p.plan_grid = L.plan_grid;
  p.plan_whole = whole_plan_ks(num_seqs, max_ctx_len, split_len, L.mtiles) > 0;
  char* ws = (char*)workspace;
  p.error_flag = (uint32_t*)(ws + L.error_off);
  p.plan = (int32_t*)(ws + L.plan_off);
  p.plan_desc = (int32_t*)(ws + L.desc_off);
  p.plan_slots = (int32_t*)(ws + L.slots_off);
  hipLaunchKernelGGL(attention_plan_kernel, dim3((unsigned)num_seqs), dim3(kHeadWaves * kWave), 0,
                     (hipStream_t)stream, p);
  return check_launch("attention_plan_kernel");
}

extern "C" int ne_paged_verify_attention_planned(
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
  AttnParams p;
  const int rc = make_params(q, q_token_stride, q_head_stride, k_cache, v_cache, k_scale, v_scale,
                             kv_dtype, scale_dtype, block_tables, block_table_stride, block_size,
                             ctx_len, q_start, q_len, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             max_q_len, max_ctx_len, softmax_scale, out, out_token_stride,
                             out_head_stride, split_len, workspace, workspace_bytes, p);
  if (rc != NE_OK) return rc;
  NE_CHECK_SUPPORTED(dma_serves(kv_dtype, scale_dtype, num_kv_heads, p.mtiles, num_seqs, k_scale, v_scale),
                     "the planned path serves 8 KV heads, at most 32 query rows per KV head and %d "
                     "sequences, and bf16 caches or int8 ones with 2-byte 4-byte-aligned scales",
                     kPlanMaxSeqs);
  // the same choice as ne_paged_attention_plan made from the same metadata
  p.plan_whole = whole_plan_ks(num_seqs, max_ctx_len, split_len, p.mtiles) > 0;
  return launch_attention_dma_for<true>(p, kv_dtype, scale_dtype, (hipStream_t)stream);
}

namespace ne {
namespace {
template <int KS, bool BF16, bool RUNS = false>
int launch_kv_stream_ks(const AttnParams& p, unsigned grid, hipStream_t s) {
  constexpr int lds = DmaShape<KS, BF16>::lds;
  static const hipError_t attr = hipFuncSetAttribute((const void*)paged_kv_stream_kernel<KS, BF16, RUNS>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) {
    set_error("paged_kv_stream_kernel: cannot reserve %d bytes of LDS: %s", lds, hipGetErrorString(attr));
    return NE_ELAUNCH;
  }
  hipLaunchKernelGGL((paged_kv_stream_kernel<KS, BF16, RUNS>), dim3(grid),
                     dim3(DmaShape<KS, BF16>::waves * kWave), lds, s, p);
  return check_launch("paged_kv_stream_kernel");
}

template <bool BF16>
int launch_kv_stream(const AttnParams& p, hipStream_t s) {
  if (p.plan_whole) {
    if (whole_plan_ks(p.num_seqs, p.max_ctx, 0, 1) == 4)
      return launch_kv_stream_ks<4, BF16>(p, (unsigned)p.num_seqs * DmaShape<4>::groups, s);
    return launch_kv_stream_ks<2, BF16>(p, (unsigned)p.num_seqs * DmaShape<2>::groups, s);
  }
  return launch_kv_stream_ks<1, BF16>(p, (unsigned)p.plan_grid, s);
}
}  // namespace
}  // namespace ne

extern "C" int ne_paged_kv_stream_planned(const void* k_cache, const void* v_cache, const void* k_scale,
                                          const void* v_scale, int32_t kv_dtype, int32_t scale_dtype,
                                          int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                                          int32_t max_q_len, int32_t max_ctx_len, int32_t split_len,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(k_cache && v_cache && workspace, "null pointer argument");
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && max_q_len > 0 &&
                   max_ctx_len > 0,
               "bad attention shape");
  NE_CHECK_ARG(kv_dtype == NE_DTYPE_BF16 || kv_dtype == NE_DTYPE_INT8, "kv_dtype must be bf16 or int8");
  NE_CHECK_ARG(split_len == 0 || (split_len > 0 && split_len % 128 == 0 && split_len <= kMaxSplitLen),
               "split_len must be 0 or a positive multiple of 128 up to %d", kMaxSplitLen);
  const Layout L = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len, kv_dtype);
  NE_CHECK_SUPPORTED(dma_serves(kv_dtype, scale_dtype, num_kv_heads, L.mtiles, num_seqs, k_scale, v_scale),
                     "the stream follows the planned path's shapes");
  NE_CHECK_ARG(workspace_bytes >= L.total, "workspace of %zu bytes is smaller than the %zu required",
               workspace_bytes, L.total);
  AttnParams p{};
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.num_seqs = num_seqs;
  p.num_kv_heads = num_kv_heads;
  p.group = L.group;
  p.mtiles = L.mtiles;
  p.max_ctx = max_ctx_len;
  p.plan_w = L.plan_w;
  p.plan_grid = L.plan_grid;
  p.plan_whole = whole_plan_ks(num_seqs, max_ctx_len, split_len, L.mtiles) > 0;
  char* ws = (char*)workspace;
  p.error_flag = (uint32_t*)(ws + L.error_off);
  p.plan = (int32_t*)(ws + L.plan_off);
  p.plan_desc = (int32_t*)(ws + L.desc_off);
  p.plan_slots = (int32_t*)(ws + L.slots_off);
  return kv_dtype == NE_DTYPE_BF16 ? launch_kv_stream<true>(p, (hipStream_t)stream)
                                   : launch_kv_stream<false>(p, (hipStream_t)stream);
}

extern "C" int ne_paged_kv_runs_plan(const int32_t* block_tables, int32_t block_table_stride, int32_t block_size,
                                     const int32_t* ctx_len, int32_t num_seqs, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t max_q_len, int32_t max_ctx_len, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
               "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads, num_kv_heads);
  NE_CHECK_SUPPORTED(block_size > 0 && block_size % kTileKeys == 0,
                     "block_size must be a positive multiple of 16 (got %d)", block_size);
  NE_CHECK_ARG(block_tables && ctx_len, "null pointer argument");
  NE_CHECK_ARG(max_q_len > 0 && max_ctx_len > 0, "max_q_len and max_ctx_len must be positive");
  const Layout L = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, 0, NE_DTYPE_INT8);
  NE_CHECK_SUPPORTED(num_kv_heads == kHeadWaves && L.mtiles <= kMaxRowTiles && num_seqs <= kPlanMaxSeqs,
                     "the runs follow the planned path's shapes: 8 KV heads, at most %d query rows per KV "
                     "head and at most %d sequences", kMaxRowTiles * kRows, kPlanMaxSeqs);
  NE_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total,
               "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
  AttnParams p{};
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.block_size = block_size;
  p.ctx_len = ctx_len;
  p.num_seqs = num_seqs;
  p.num_kv_heads = num_kv_heads;
  p.max_ctx = max_ctx_len;
  p.plan_grid = L.plan_grid;
  char* ws = (char*)workspace;
  p.error_flag = (uint32_t*)(ws + L.error_off);
  p.plan_desc = (int32_t*)(ws + L.desc_off);
  p.plan_slots = (int32_t*)(ws + L.slots_off);
  hipLaunchKernelGGL(kv_runs_plan_kernel, dim3((unsigned)L.plan_grid), dim3(kHeadWaves * kWave), 0,
                     (hipStream_t)stream, p);
  return check_launch("kv_runs_plan_kernel");
}

extern "C" int ne_paged_kv_stream_runs(const void* k_cache, const void* v_cache, const void* k_scale,
                                       const void* v_scale, int32_t kv_dtype, int32_t scale_dtype, int32_t num_seqs,
                                       int32_t num_q_heads, int32_t num_kv_heads, int32_t max_q_len,
                                       int32_t max_ctx_len, void* workspace, size_t workspace_bytes, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(k_cache && v_cache && workspace, "null pointer argument");
  NE_CHECK_ARG(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && max_q_len > 0 &&
                   max_ctx_len > 0,
               "bad attention shape");
  NE_CHECK_ARG(kv_dtype == NE_DTYPE_BF16 || kv_dtype == NE_DTYPE_INT8, "kv_dtype must be bf16 or int8");
  const Layout L = make_layout(num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, 0, kv_dtype);
  NE_CHECK_SUPPORTED(dma_serves(kv_dtype, scale_dtype, num_kv_heads, L.mtiles, num_seqs, k_scale, v_scale),
                     "the stream follows the planned path's shapes");
  NE_CHECK_ARG(workspace_bytes >= L.total, "workspace of %zu bytes is smaller than the %zu required",
               workspace_bytes, L.total);
  AttnParams p{};
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.num_seqs = num_seqs;
  p.num_kv_heads = num_kv_heads;
  p.max_ctx = max_ctx_len;
  p.plan_grid = L.plan_grid;
  char* ws = (char*)workspace;
  p.error_flag = (uint32_t*)(ws + L.error_off);
  p.plan_desc = (int32_t*)(ws + L.desc_off);
  p.plan_slots = (int32_t*)(ws + L.slots_off);
  return kv_dtype == NE_DTYPE_BF16
             ? launch_kv_stream_ks<1, true, true>(p, (unsigned)L.plan_grid, (hipStream_t)stream)
             : launch_kv_stream_ks<1, false, true>(p, (unsigned)L.plan_grid, (hipStream_t)stream);
}
