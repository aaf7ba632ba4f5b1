// W8A16 projection GEMMs and the bf16 LM-head GEMM for gfx950.
//
// Replaces Int8Linear.forward (ne/models/int8_quantization.py:55-57), which
// materialises bf16(int8 * scale) for the whole weight before F.linear, and the
// tied-embedding LM head (ne/models/qwen3.py:197-203).
//
// Shapes here are short and wide: M = query rows of a verify step (64 x 5 =
// 320), N up to 6144 (151936 for the LM head), K 1024..3072.  Both kernels stage
// X and W tiles in LDS with DMA copies (global_load_lds_dwordx4) so that copies
// stay in flight while the MFMAs (v_mfma_f32_16x16x32_bf16) consume the previous
// stage.  Each MFMA computes D = W . X^T (weight rows x token rows), so a lane ends
// up holding four consecutive output columns of one token row (8-byte stores).
// int8 weights become bf16 in registers after the LDS read (exact); the per-row
// scale is applied to the fp32 sum.
//
// At M = 320 every N-tile re-reads X; the tiles are sized to keep that traffic per CU
// near its minimum for 256 independent tiles, and the LM head keeps all 320 rows
// resident per work-group to read X once per 256 columns.  A projection's time is its
// work-group's chain (first weight fetch from HBM, then per stage a barrier, the copy
// issue, the fragment reads and the MFMAs, then the k-group exchange), not L2 -> CU
// bandwidth (~30 TB/s with enough loads in flight), HBM or the MFMAs.
#include "ne_common.hpp"
#include "qk_rope_kv.hpp"

namespace ne {

namespace {

struct GemmParams {
  const uint16_t* x;
  int64_t ldx;
  const void* w;
  const void* scale;
  int m, n, k;
  uint16_t* y;
  int64_t ldy;
  uint64_t* argmax;  // [m][n / BN] packed (ordered value, ~index)
  int tiles_m, tiles_n;
};

__device__ __forceinline__ float sbyte(uint32_t w, int k) { return (float)(int8_t)(w >> (8 * k)); }

__device__ __forceinline__ bf16x8 int8x8_to_bf16x8(uint32_t a, uint32_t b) {
  u32x4 r = {pack_bf16x2(sbyte(a, 0), sbyte(a, 1)), pack_bf16x2(sbyte(a, 2), sbyte(a, 3)),
             pack_bf16x2(sbyte(b, 0), sbyte(b, 1)), pack_bf16x2(sbyte(b, 2), sbyte(b, 3))};
  return __builtin_bit_cast(bf16x8, r);
}

// order-preserving key: larger value wins, then smaller index wins
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  v = v + 0.0f;  // -0 compares equal to +0 (torch.argmax): give both one key
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((uint32_t)v, o);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o);
  return ((uint64_t)hi << 32) | lo;
}

template <int SDT>
__device__ __forceinline__ float scale_at(const void* s, int64_t i) {
  if constexpr (SDT < 0) {
    return 1.f;
  } else {
    return load_scale<SDT>(s, i);
  }
}

// ---- shared pieces -------------------------------------------------------------
// Tiles are copied global -> LDS with global_load_lds_dwordx4: every wave-instruction
// copies 1 KiB of whole 128-byte lines (4 rows of 256 B or 8 rows of 128 B), the access
// shape the vector L1 serves at full rate.  Each lane picks its source so that LDS row
// `row` holds 16-byte chunk c at position c ^ (row % chunks-per-row), which makes the
// MFMA fragment reads bank-conflict free.
constexpr int kArgmaxCols = 64;  // columns per LM-head argmax partial
constexpr int kStageK = 128;     // k per stage of the projection kernel
// the projection kernels address X rows with 32-bit byte offsets from a scalar base
constexpr int64_t kMaxXElems = (int64_t(1) << 31) - 256;

__device__ __forceinline__ void lds_dma16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_wave_base, 16,
                                   0, 0);
}

// s_waitcnt vmcnt(n) leaving lgkmcnt/expcnt unconstrained (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---- W8A16 projections ----------------------------------------------------------
// Work-group tile: PM * 16 token rows (80 for the plain shapes, 48 for split-K) x 16 *
// NSUB weight rows, sized so that the verify-step shapes give about one work-group per
// CU (M = 320: QKV N = 4096 and gate|up N = 6144 give 256 tiles; o / down N = 1024 give
// 7 x 16 tiles of 48 rows, split 2 ways over K).  For o / down, 48-row tiles and two
// splits (224 work-groups) against 80-row tiles and four (256): the split-K sum +
// RMSNorm that follows reads half the fp32 partials; with 28 distinct weights replayed
// back to back the pair takes 9.5 / 10.6 us instead of 10.6 / 11.3 us, inside the
// verify step the GEMMs take the same time and the norm 0.14 us less.  Fewer rows gain
// more: 288 rows (6 x 16 x 2 work-groups instead of 4 x 16 x 4) and 64 rows (2 x 16 x 4
// instead of 1 x 16 x 4).  The MFMA waves form KG k-groups x NSUB / NPW: wave (kg, nw) runs the
// 4 / KG k-steps kg * 4 / KG .. (32 wide each) of every 128-wide stage for all PM token
// subtiles against weight subtiles nw * NPW .. + NPW, so each X fragment read from LDS
// feeds NPW MFMAs and each weight fragment PM.  At the end, wave (kg, nw) finishes the
// token subtiles mi with mi % KG == kg: the other k-groups' partial tiles of those come
// through LDS and are added in k-group order.  Two k-groups halve that exchange (and
// its barrier wait) against four, for twice the X fragment reads in the loop.
//
// Stages are copied by DMA into two LDS rings: X rows (from L2, where every column
// tile re-reads them) run kRX - 1 stages ahead and weight rows (from HBM, the longer
// way) kRW - 1 stages ahead.  A wave copies either X or weight rows, never both, so
// its vmcnt counts one stream and its wait for a stage is exact.  Each wave reads the
// fragments of stage t from LDS before it runs the MFMAs of stage t - 1 (held in
// registers), so the LDS latency hides under the multiplies.
constexpr int kPM = 5;       // token subtiles per work-group (the fused QKV epilogue uses 3)
constexpr int kSplitPM = 3;  // token subtiles per work-group of the split-K product
constexpr int kQkvKRows = 32;  // rows per work-group of the fused QKV kernel's k heads (q / v: 48)

template <int NSUB, int PM, int KG, int NPW>
struct ProjLayout {
  static_assert(KG == 1 || KG == 2 || KG == 4, "k-groups split the 4 k-steps of a stage");
  static_assert(NSUB % NPW == 0, "weight subtiles per wave");
  static constexpr int kKS = 4 / KG;  // k-steps per wave per stage
  static constexpr int kPRows = PM * 16;
  static constexpr int kNW = NSUB / NPW;
  static constexpr int kWaves = KG * kNW;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kXI = PM * 4;    // 1 KiB copies per stage: X rows of 256 B ...
  static constexpr int kWI = NSUB * 2;  // ... and weight rows of 128 B
  static constexpr int kXBytes = kXI * 1024;
  static constexpr int kWBytes = kWI * 1024;
  static constexpr int kRX = 3;
  static constexpr int kRW = 6;
  // copies per X-copying / weight-copying wave: the fewest per wave that fit the waves
  static constexpr int split() {
    int best = -1, cost = 1 << 30;
    for (int dx = 1; dx <= kXI; ++dx)
      for (int dw = 1; dw <= kWI; ++dw)
        if (kXI % dx == 0 && kWI % dw == 0 && kXI / dx + kWI / dw <= kWaves && (dx > dw ? dx : dw) < cost) {
          cost = dx > dw ? dx : dw;
          best = dx * 256 + dw;
        }
    return best;
  }
  static constexpr int kDX = split() / 256;
  static constexpr int kDW = split() % 256;
  static constexpr int kNXW = kXI / kDX;  // waves [0, kNXW) copy X
  static constexpr int kNWW = kWI / kDW;  // waves [kNXW, kNXW + kNWW) copy weights
  static constexpr int kRedBytes = KG * kNW * PM * NPW * 1024;
  static constexpr int kRing = kRX * kXBytes + kRW * kWBytes;
  static constexpr int kLds = kRing > kRedBytes ? kRing : kRedBytes;
  static_assert(split() > 0, "copy split");
  static_assert(kDX * (kRX - 2) < 64 && kDW * (kRW - 2) < 64, "vmcnt range");
  static_assert(kLds <= 160 * 1024, "LDS");
};

// a wave-uniform pointer kept in SGPRs, so that a copy's address is a scalar base plus
// a 32-bit lane offset
__device__ __forceinline__ const char* uniform_ptr(const char* ptr) {
  const uint64_t v = (uint64_t)ptr;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const char*)(((uint64_t)hi << 32) | lo);
}

// s_waitcnt vmcnt(D * pend) for a run-time pend in [0, P]
template <int D, int P>
__device__ __forceinline__ void wait_pending(int pend) {
  if constexpr (P <= 0) {
    wait_vmcnt<0>();
  } else {
    if (pend >= P) {
      wait_vmcnt<D * P>();
    } else {
      wait_pending<D, P - 1>(pend);
    }
  }
}

__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// The k loop of a work-group: kt_n stages of 128 from k = kbase (KT > 0: kt_n = KT).  X rows m0.. (rows past
// m re-read row m - 1 and are never stored) and weight rows n0.. are copied with the
// chunk swizzles below; in k-step kk (0..3) of a stage, lane group g = lane / 16
// supplies logical k = 64 (kk / 2) + 16 g + 8 (kk % 2) + e, e < 8: X chunk
// 8 (kk / 2) + 2 g + kk % 2 of its 256-byte row, weight bytes 16 (4 (kk / 2) + g) +
// 8 (kk % 2) of its 128-byte row.  Wave (kg, nw) runs k-steps kk = kg * KS + s.
template <int NSUB, int PM, int KG, int NPW, int KT>
__device__ __forceinline__ void proj_mainloop(const GemmParams& p, char* smem, int m0, int n0, int kbase,
                                              int kt_runtime, int wave, int lane, int kg, int nw,
                                              floatx4 (&acc)[PM][NPW]) {
  using L = ProjLayout<NSUB, PM, KG, NPW>;
  constexpr int KS = L::kKS;
  // a stage count known at compile time turns every wait below into one instruction
  const int kt_n = KT > 0 ? KT : kt_runtime;
  const int r = lane & 15;
  const int g = lane >> 4;
  const bool xwave = wave < L::kNXW;
  const bool wwave = wave >= L::kNXW && wave < L::kNXW + L::kNWW;
  constexpr int D = L::kDX > L::kDW ? L::kDX : L::kDW;
  // copy j of this wave: LDS position c ^ (row % chunks-per-row) for 16-byte chunk c of
  // LDS row `row`, which makes the fragment reads bank-conflict free
  uint32_t off[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    if (xwave) {  // 4 X rows x 16 chunks
      const int row = (wave * L::kDX + j) * 4 + (lane >> 4);
      const int chunk = (lane & 15) ^ (row & 15);
      const int grow = min(m0 + row, p.m - 1);
      off[j] = (uint32_t)grow * (uint32_t)(p.ldx * 2) + (uint32_t)chunk * 16u;
    } else {  // 8 weight rows x 8 chunks
      const int row = ((wave - L::kNXW) * L::kDW + j) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ (row & 7);
      off[j] = (uint32_t)row * (uint32_t)p.k + (uint32_t)chunk * 16u;
    }
  }
  const char* xbase = (const char*)p.x + (int64_t)kbase * 2;
  const char* wbase = (const char*)p.w + (int64_t)n0 * p.k + kbase;
  char* xring = smem;
  char* wring = smem + L::kRX * L::kXBytes;
  auto issue_x = [&](int s) {
    if (!xwave) return;
    char* slot = xring + (s % L::kRX) * L::kXBytes + wave * L::kDX * 1024;
    const char* src = uniform_ptr(xbase + s * (kStageK * 2));
#pragma unroll
    for (int j = 0; j < L::kDX; ++j) {
      uint32_t o = off[j];
      __asm__("" : "+v"(o));  // keep the lane offset 32-bit: scalar base + offset addressing
      lds_dma16(src + o, slot + j * 1024);
    }
  };
  auto issue_w = [&](int s) {
    if (!wwave) return;
    char* slot = wring + (s % L::kRW) * L::kWBytes + (wave - L::kNXW) * L::kDW * 1024;
    const char* src = uniform_ptr(wbase + s * kStageK);
#pragma unroll
    for (int j = 0; j < L::kDW; ++j) {
      uint32_t o = off[j];
      __asm__("" : "+v"(o));
      lds_dma16(src + o, slot + j * 1024);
    }
  };
  // stage t needs this wave's copies of stage t; those of later stages may still fly
  auto wait_stage = [&](int t) {
    if (xwave) wait_pending<L::kDX, L::kRX - 2>(min(kt_n - t - 1, L::kRX - 2));
    if (wwave) wait_pending<L::kDW, L::kRW - 2>(min(kt_n - t - 1, L::kRW - 2));
  };
  uint32_t xr[KS], wr[KS];
#pragma unroll
  for (int q = 0; q < KS; ++q) {
    const int kk = kg * KS + q;
    const int cx = 8 * (kk >> 1) + 2 * g + (kk & 1);
    xr[q] = (uint32_t)(r * 256 + ((cx ^ r) * 16));
    const int cw = 4 * (kk >> 1) + g;
    wr[q] = (uint32_t)((nw * NPW * 16 + r) * 128 + ((cw ^ (r & 7)) * 16) + (kk & 1) * 8);
  }
  using XFrag = u32x4[KS][PM];
  using WFrag = u32x2[KS][NPW];
  using AFrag = bf16x8[KS][NPW];
  // weight fragments first: their conversion is the first thing waiting on them
  auto read = [&](int s, XFrag& xf, WFrag& wf) {
    const char* xs = xring + (s % L::kRX) * L::kXBytes;
    const char* ws = wring + (s % L::kRW) * L::kWBytes;
#pragma unroll
    for (int q = 0; q < KS; ++q)
#pragma unroll
      for (int ns = 0; ns < NPW; ++ns) wf[q][ns] = *(const u32x2*)(ws + wr[q] + ns * 2048);
#pragma unroll
    for (int q = 0; q < KS; ++q)
#pragma unroll
      for (int mi = 0; mi < PM; ++mi) xf[q][mi] = *(const u32x4*)(xs + xr[q] + mi * 4096);
  };
  auto convert = [&](const WFrag& wf, AFrag& a) {
#pragma unroll
    for (int q = 0; q < KS; ++q)
#pragma unroll
      for (int ns = 0; ns < NPW; ++ns) a[q][ns] = int8x8_to_bf16x8(wf[q][ns][0], wf[q][ns][1]);
  };
  auto mma = [&](const XFrag& xf, const AFrag& a) {
#pragma unroll
    for (int q = 0; q < KS; ++q)
#pragma unroll
      for (int mi = 0; mi < PM; ++mi)
#pragma unroll
        for (int ns = 0; ns < NPW; ++ns)
          acc[mi][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[q][ns], __builtin_bit_cast(bf16x8, xf[q][mi]),
                                                                acc[mi][ns], 0, 0, 0);
  };
  // stage t: its copies are in LDS after the barrier, and every wave has read stage
  // t - 1 into registers before it (lgkmcnt(0)), so the slots of stage t - 1 take the
  // copies of stages t + kRX - 1 and t + kRW - 1.  The MFMAs of stage t - 1 run on
  // weights converted to bf16 from the int8 read in step t - 1; the compiler places that
  // conversion just before those MFMAs (it keeps the int8 form live across the barrier),
  // so a wave converts and then multiplies.
  auto step = [&](int t, XFrag& xr_, WFrag& wr_, AFrag& ar, const XFrag& xm, const AFrag& am) {
    wait_stage(t);
    wait_lgkmcnt0();
    asm volatile("s_barrier" ::: "memory");
    if (t + L::kRX - 1 < kt_n) issue_x(t + L::kRX - 1);
    if (t + L::kRW - 1 < kt_n) issue_w(t + L::kRW - 1);
    read(t, xr_, wr_);
    __builtin_amdgcn_sched_barrier(0);  // the reads go out before the multiplies
    mma(xm, am);
    convert(wr_, ar);
    __builtin_amdgcn_sched_barrier(0);
  };

#pragma unroll
  for (int s = 0; s < L::kRW - 1; ++s)
    if (s < kt_n) issue_w(s);  // the weights first: they have the longer way to come
#pragma unroll
  for (int s = 0; s < L::kRX - 1; ++s)
    if (s < kt_n) issue_x(s);
  XFrag xa, xb;
  WFrag wa, wb;
  AFrag aa, ab;
  wait_stage(0);
  asm volatile("s_barrier" ::: "memory");
  if (L::kRX - 1 < kt_n) issue_x(L::kRX - 1);
  if (L::kRW - 1 < kt_n) issue_w(L::kRW - 1);
  read(0, xa, wa);
  convert(wa, aa);
  int t = 1;
  for (; t + 1 < kt_n; t += 2) {
    step(t, xb, wb, ab, xa, aa);
    step(t + 1, xa, wa, aa, xb, ab);
  }
  if (t < kt_n) {
    step(t, xb, wb, ab, xa, aa);
    wait_lgkmcnt0();
    mma(xb, ab);
  } else {
    wait_lgkmcnt0();
    mma(xa, aa);
  }
}

// EPI 0: y = bf16(acc * scale); 1: SwiGLU of paired gate/up subtiles; 3: fp32 partial
// sums of K split blockIdx.y, scaled, into partial[split][m][n]; 4: the QKV projection
// with one 128-column head per tile (NSUB 8), each head vector of the bf16 result taken
// through QK-norm + RoPE into q_out or quantised into the KV cache (qk_rope_kv.hpp) --
// the bits the GEMM with EPI 0 followed by the row kernel produce, without the qkv round
// trip through memory.  KV (EPI 4): 1 bf16 cache, 2 int8 + bf16 scales, 3 int8 + fp16.
template <int NSUB, int SDT, int EPI, int KV, int PM, int KG, int NPW, int KT>
__global__ __launch_bounds__((ProjLayout<NSUB, PM, KG, NPW>::kThreads)) void proj_kernel(
    GemmParams p, int k_per_split, float* partial, QkvRopeArgs qa) {
  using L = ProjLayout<NSUB, PM, KG, NPW>;
  constexpr int kPRows = L::kPRows;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // Every kernel argument the work-group uses, requested in one batch: left to itself
  // the compiler loads each next to its first use, and the tile index, the copy
  // addresses and the epilogue then wait on one scalar-cache round trip after another.
  asm volatile("" ::"s"(p.x), "s"(p.ldx), "s"(p.w), "s"(p.scale), "s"(p.m), "s"(p.k), "s"(p.tiles_m),
               "s"(p.tiles_n), "s"(k_per_split));
  if constexpr (EPI == 3) {
    asm volatile("" ::"s"(partial), "s"(p.n));
  } else if constexpr (EPI != 4) {
    asm volatile("" ::"s"(p.y), "s"(p.ldy));
  } else {
    asm volatile("" ::"s"(qa.q_norm_w), "s"(qa.k_norm_w), "s"(qa.positions), "s"(qa.slot_mapping),
                 "s"(qa.rope), "s"(qa.rope_positions), "s"(qa.hq));
  }
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int jj = bid / kNumXcd;
  int tm = jj % p.tiles_m;
  int tn = (jj / p.tiles_m) * kNumXcd + xcd;  // the M tiles of one weight tile share an XCD
  int tile_rows = kPRows;
  if constexpr (EPI == 4) {
    // heads xcd, xcd + 8, ... on this XCD, each with all its row tiles: kPRows rows for
    // q / v heads, kQkvKRows for k heads (whose epilogue also quantises, so fewer rows
    // per work-group even out the work-groups' end times)
    int j = jj;
    tn = -1;
    for (int h = xcd; h < p.tiles_n; h += kNumXcd) {
      const bool kh = h >= qa.hq && h < qa.hq + qa.hkv;
      const int t = kh ? qa.tiles_k : p.tiles_m;
      if (j < t) {
        tn = h;
        tm = j;
        tile_rows = kh ? kQkvKRows : kPRows;
        break;
      }
      j -= t;
    }
    if (tn < 0) return;
  }
  if (tn >= p.tiles_n) return;
  const int split = blockIdx.y;
  const int m0 = tm * tile_rows;
  const int n0 = tn * NSUB * 16;
  const int kbase = split * k_per_split;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int kg = wave / L::kNW;
  const int nw = wave % L::kNW;
  const int r = lane & 15;
  const int g = lane >> 4;

  // the epilogue's weight-row scales, fetched now so that their latency hides under
  // the k loop: lane (r, g) stores columns (nw NPW + ns) 16 + 4 g + i
  float sc[NPW][4] = {};
  if constexpr (EPI != 4) {  // EPI 4 scales its rows' columns instead (e_sc)
#pragma unroll
    for (int ns = 0; ns < NPW; ++ns)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[ns][i] = scale_at<SDT>(p.scale, n0 + (nw * NPW + ns) * 16 + 4 * g + i);
  }

  // EPI 4: wave w finishes rows w, w + kWaves, ... of the tile (head tn).  Their slots
  // and positions (scalar loads) and the head's norm weights are requested now and
  // used only in the epilogue, so no wait for them precedes the k loop; the RoPE
  // values, which need the positions, are requested right after the k loop.
  constexpr int kEpiRows = (kPRows + L::kWaves - 1) / L::kWaves;
  int e_slot[kEpiRows], e_pos[kEpiRows];
  uint16_t e_w[2] = {0, 0};
  float e_sc[2] = {0.f, 0.f};  // weight-row scales of head columns lane and lane + 64
  if constexpr (EPI == 4) {
    const uint16_t* w = (tn < qa.hq) ? qa.q_norm_w : qa.k_norm_w;  // v heads do not use it
    e_w[0] = w[lane];
    e_w[1] = w[lane + 64];
    e_sc[0] = scale_at<SDT>(p.scale, n0 + lane);
    e_sc[1] = scale_at<SDT>(p.scale, n0 + 64 + lane);
#pragma unroll
    for (int i = 0; i < kEpiRows; ++i) {
      const int m = min(m0 + wave + L::kWaves * i, p.m - 1);
      e_slot[i] = ((const ConstI32*)qa.slot_mapping)[m];
      e_pos[i] = ((const ConstI32*)qa.positions)[m];
    }
  }

  floatx4 acc[PM][NPW];
#pragma unroll
  for (int mi = 0; mi < PM; ++mi)
#pragma unroll
    for (int ns = 0; ns < NPW; ++ns) acc[mi][ns] = floatx4{0.f, 0.f, 0.f, 0.f};

  proj_mainloop<NSUB, PM, KG, NPW, KT>(p, smem, m0, n0, kbase, k_per_split / kStageK, wave, lane, kg, nw,
                                       acc);

  // EPI 4: the rows' cos / sin, in flight while the k-groups are summed
  uint16_t e_rc[kEpiRows], e_rs[kEpiRows];
  if constexpr (EPI == 4) {
    // the loads issued before the k loop are long done: take their values now, so that
    // the compiler's wait for them does not land after the loads below
    __asm__ __volatile__("" ::"v"(e_sc[0]), "v"(e_sc[1]), "v"(e_w[0]), "v"(e_w[1]));
#pragma unroll
    for (int i = 0; i < kEpiRows; ++i) {
      const int64_t pos = min(max(e_pos[i], 0), qa.rope_positions - 1);
      e_rc[i] = qa.rope[pos * 128 + lane];
      e_rs[i] = qa.rope[pos * 128 + 64 + lane];
    }
  }

  // ---- sum the k-groups through LDS (the stage ring is free once all waves pass) ----
  lds_barrier();
  if constexpr (EPI == 4) {
    // partials as rows [kg][row][128 + 4 pad] fp32, so that the row pass below reads a
    // row's columns lane and lane + 64 as consecutive words; each row is summed over the
    // k-groups in order and scaled, the bits the GEMM epilogue stores
    static_assert(NSUB == 8, "one head per tile");
    constexpr int kRowF = 132;
    static_assert(KG * kPRows * kRowF * 4 <= L::kLds, "partials fit the stage ring");
    constexpr bool kInt8 = KV >= 2;
    constexpr int kKvSdt = KV == 3 ? NE_DTYPE_FP16 : NE_DTYPE_BF16;
    float* part = (float*)smem;
#pragma unroll
    for (int mi = 0; mi < PM; ++mi)
#pragma unroll
      for (int ns = 0; ns < NPW; ++ns)
        *(floatx4*)(part + (kg * kPRows + mi * 16 + r) * kRowF + (nw * NPW + ns) * 16 + 4 * g) = acc[mi][ns];
    lds_barrier();
    // this wave's rows all at once, so that their reductions overlap
    auto rows_pass = [&](auto n_rows) {
      constexpr int N = decltype(n_rows)::value;
      int rows_e[N];
      bool valid_e[N];
      float a_e[N], b_e[N], c_e[N], s_e[N];
      int64_t slot_e[N];
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int rr = min(wave + L::kWaves * i, kPRows - 1);
        rows_e[i] = m0 + rr;
        valid_e[i] = wave + L::kWaves * i < tile_rows && m0 + rr < p.m;
        float va = part[rr * kRowF + lane];
        float vb = part[rr * kRowF + 64 + lane];
#pragma unroll
        for (int q = 1; q < KG; ++q) {
          va += part[(q * kPRows + rr) * kRowF + lane];
          vb += part[(q * kPRows + rr) * kRowF + 64 + lane];
        }
        a_e[i] = bf16_round(va * e_sc[0]);
        b_e[i] = bf16_round(vb * e_sc[1]);
        c_e[i] = bf16_to_f32(e_rc[i]);
        s_e[i] = bf16_to_f32(e_rs[i]);
        slot_e[i] = e_slot[i];
      }
      qk_norm_rope_kv_vectors<kInt8, kKvSdt, N>(qa, rows_e, valid_e, tn, lane, a_e, b_e, slot_e,
                                                bf16_to_f32(e_w[0]), bf16_to_f32(e_w[1]), c_e, s_e);
    };
    static_assert(kQkvKRows % L::kWaves == 0 && kQkvKRows / L::kWaves <= kEpiRows, "k-tile rows per wave");
    if (tile_rows == kQkvKRows) {
      rows_pass(std::integral_constant<int, kQkvKRows / L::kWaves>{});
    } else {
      rows_pass(std::integral_constant<int, kEpiRows>{});
    }
    return;
  }
  // Token subtile mi is finished by k-group mi % KG: each wave hands the partial tiles of
  // the other subtiles to their finishing wave through LDS, [kg][nw][mi][ns][lane].
  floatx4* red = (floatx4*)smem;
  auto red_at = [&](int q, int mi, int ns) -> floatx4& {
    return red[(((q * L::kNW + nw) * PM + mi) * NPW + ns) * kWave + lane];
  };
#pragma unroll
  for (int mi = 0; mi < PM; ++mi)
    if (KG > 1 && mi % KG != kg)
#pragma unroll
      for (int ns = 0; ns < NPW; ++ns) red_at(kg, mi, ns) = acc[mi][ns];
  if constexpr (KG > 1) lds_barrier();

#pragma unroll
  for (int mi = 0; mi < PM; ++mi) {
    if (mi % KG != kg) continue;
    floatx4 v[NPW];
#pragma unroll
    for (int ns = 0; ns < NPW; ++ns) {
      // in k-group order, this wave's own partial from its registers
      v[ns] = kg == 0 ? acc[mi][ns] : red_at(0, mi, ns);
#pragma unroll
      for (int q = 1; q < KG; ++q) v[ns] += q == kg ? acc[mi][ns] : red_at(q, mi, ns);
    }
    // lane holds D[n = 4 g + i][m = r] of weight subtiles nw NPW + ns
    const int m = m0 + mi * 16 + r;
    if (m >= p.m) continue;
    if constexpr (EPI == 0) {
#pragma unroll
      for (int ns = 0; ns < NPW; ++ns) {
        const int n = n0 + (nw * NPW + ns) * 16 + 4 * g;
        const u32x2 bits = {pack_bf16x2(v[ns][0] * sc[ns][0], v[ns][1] * sc[ns][1]),
                            pack_bf16x2(v[ns][2] * sc[ns][2], v[ns][3] * sc[ns][3])};
        *(u32x2*)(p.y + (int64_t)m * p.ldy + n) = bits;
      }
    } else if constexpr (EPI == 1) {
      static_assert(NPW == 2, "a wave holds paired gate / up subtiles");
      float out[4];  // gate rows are subtile 2 nw, the paired up rows subtile 2 nw + 1
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gate = bf16_round(v[0][i] * sc[0][i]);
        const float up = bf16_round(v[1][i] * sc[1][i]);
        const float silu = bf16_round(gate / (1.f + __expf(-gate)));
        out[i] = silu * up;
      }
      const int ncol = (n0 + 2 * nw * 16) / 2 + 4 * g;
      const u32x2 bits = {pack_bf16x2(out[0], out[1]), pack_bf16x2(out[2], out[3])};
      *(u32x2*)(p.y + (int64_t)m * p.ldy + ncol) = bits;
    } else {
#pragma unroll
      for (int ns = 0; ns < NPW; ++ns) {
        const int n = n0 + (nw * NPW + ns) * 16 + 4 * g;
        const floatx4 sv = {v[ns][0] * sc[ns][0], v[ns][1] * sc[ns][1], v[ns][2] * sc[ns][2],
                            v[ns][3] * sc[ns][3]};
        *(floatx4*)(partial + ((int64_t)split * p.m + m) * p.n + n) = sv;
      }
    }
  }
}

template <int NSUB, int SDT, int EPI, int KV, int PM, int KG, int NPW, int KT>
int launch_proj_kt(GemmParams p, int splits, float* partial, hipStream_t stream, const char* name,
                   QkvRopeArgs qa) {
  using L = ProjLayout<NSUB, PM, KG, NPW>;
  p.tiles_m = ceil_div(p.m, L::kPRows);
  p.tiles_n = p.n / (NSUB * 16);
  const int tiles_n_padded = ceil_div(p.tiles_n, kNumXcd) * kNumXcd;
  dim3 grid((unsigned)(p.tiles_m * tiles_n_padded), (unsigned)splits);
  if constexpr (EPI == 4) {
    // per XCD: its heads' row tiles (k heads in tiles of kQkvKRows); the grid covers the
    // XCD with the most
    qa.tiles_k = ceil_div(p.m, kQkvKRows);
    int most = 0;
    for (int x = 0; x < kNumXcd; ++x) {
      int t = 0;
      for (int h = x; h < p.tiles_n; h += kNumXcd) t += (h >= qa.hq && h < qa.hq + qa.hkv) ? qa.tiles_k : p.tiles_m;
      most = t > most ? t : most;
    }
    grid.x = (unsigned)(most * kNumXcd);
  }
  static const hipError_t attr = hipFuncSetAttribute(
      (const void*)proj_kernel<NSUB, SDT, EPI, KV, PM, KG, NPW, KT>, hipFuncAttributeMaxDynamicSharedMemorySize,
      L::kLds);
  if (attr != hipSuccess) {
    set_error("%s: cannot reserve %d bytes of LDS: %s", name, L::kLds, hipGetErrorString(attr));
    return NE_ELAUNCH;
  }
  hipLaunchKernelGGL((proj_kernel<NSUB, SDT, EPI, KV, PM, KG, NPW, KT>), grid, dim3(L::kThreads), L::kLds,
                     stream, p, p.k / splits, partial, qa);
  return check_launch(name);
}

// Stage counts with a kernel of their own: 8 (K = 1024, the QKV and gate|up
// projections of the 0.6B model), and for split-K 8 and 12 (o and down split 2 ways over
// K = 2048 and 3072) and 4 and 6 (the same split 4 ways, for fewer rows); any other
// count runs the loop with a run-time count.
template <int NSUB, int SDT, int EPI, int KV, int PM, int KG, int NPW>
int launch_proj(GemmParams p, int splits, float* partial, hipStream_t stream, const char* name,
                const QkvRopeArgs& qa = QkvRopeArgs{}) {
  const int kt = p.k / splits / kStageK;
  if constexpr (EPI == 3) {
    if (kt == 4) return launch_proj_kt<NSUB, SDT, EPI, KV, PM, KG, NPW, 4>(p, splits, partial, stream, name, qa);
    if (kt == 6) return launch_proj_kt<NSUB, SDT, EPI, KV, PM, KG, NPW, 6>(p, splits, partial, stream, name, qa);
    if (kt == 8) return launch_proj_kt<NSUB, SDT, EPI, KV, PM, KG, NPW, 8>(p, splits, partial, stream, name, qa);
    if (kt == 12) return launch_proj_kt<NSUB, SDT, EPI, KV, PM, KG, NPW, 12>(p, splits, partial, stream, name, qa);
  } else {
    if (kt == 8) return launch_proj_kt<NSUB, SDT, EPI, KV, PM, KG, NPW, 8>(p, splits, partial, stream, name, qa);
  }
  return launch_proj_kt<NSUB, SDT, EPI, KV, PM, KG, NPW, 0>(p, splits, partial, stream, name, qa);
}

// Wave layouts (k-groups, weight subtiles per wave).  The plain and split-K products and
// the fused QKV projection share two k-groups, so the fused epilogue sums every output in
// the order the plain GEMM does and both round to the same bits; SwiGLU pairs gate and
// up subtiles in one wave and keeps four k-groups to keep 12 waves.
constexpr int kKgPlain = 2, kNpwPlain = 1;
constexpr int kKgQkv = 2, kNpwQkv = 2;
constexpr int kKgSwiglu = 4, kNpwSwiglu = 2;

template <int SDT>
int dispatch_qkv_fused(GemmParams p, const QkvRopeArgs& qa, int kv_mode, hipStream_t s) {
  switch (kv_mode) {
    // 48-row tiles: 7 x 32 = 224 work-groups for 320 rows, 3 rows per wave in the epilogue
    case 1: return launch_proj<8, SDT, 4, 1, 3, kKgQkv, kNpwQkv>(p, 1, nullptr, s, "w8a16_qkv_norm_rope_kv", qa);
    case 2: return launch_proj<8, SDT, 4, 2, 3, kKgQkv, kNpwQkv>(p, 1, nullptr, s, "w8a16_qkv_norm_rope_kv", qa);
    default: return launch_proj<8, SDT, 4, 3, 3, kKgQkv, kNpwQkv>(p, 1, nullptr, s, "w8a16_qkv_norm_rope_kv", qa);
  }
}

template <int SDT>
int dispatch_w8a16(GemmParams p, int epilogue, int splits, float* partial, hipStream_t s) {
  if (epilogue == NE_EPILOGUE_SWIGLU) {
    if (p.n % 96 == 0)
      return launch_proj<6, SDT, 1, 0, kPM, kKgSwiglu, kNpwSwiglu>(p, 1, nullptr, s, "w8a16_swiglu");
    return launch_proj<4, SDT, 1, 0, kPM, kKgSwiglu, kNpwSwiglu>(p, 1, nullptr, s, "w8a16_swiglu");
  }
  if (partial != nullptr)
    return launch_proj<4, SDT, 3, 0, kSplitPM, kKgPlain, kNpwPlain>(p, splits, partial, s, "w8a16_splitk");
  return launch_proj<4, SDT, 0, 0, kPM, kKgPlain, kNpwPlain>(p, 1, nullptr, s, "w8a16_gemm");
}

// ---- LM head: persistent work-groups over the vocabulary -------------------------
// logits = X . W^T for X [m, k] bf16 and the tied embedding W [vocab, k] bf16, plus
// argmax partials: per row, one (value, index) key for each half of each work-group's
// column range (the range's 128-column halves of every block, kept as a running
// maximum, so that the acceptance kernel reduces 512 keys per row, not one per 64
// columns).  Inside the kernel a key is 32 bits: a 16-bit order code of the bf16 value
// over 16 bits of column within the range.  The weight (311 MB for 151936 x 1024) is
// read from HBM once; what limits a tiled GEMM at m = 320 is the L2 -> CU traffic
// of X, which every column tile re-reads (about 2.3 GB over 64 x 128 tiles).  So
// one work-group per CU owns a contiguous range of 64-column groups and walks it in
// blocks of 256 columns against all rows at once: 8 waves, wave (mw, nw) holding
// rows 80 mw .. +80 and columns 128 nw .. +128 of the block in 160 accumulators,
// which cuts the X traffic to one read per 256 columns.  K advances in stages of 64
// (X 40 KiB + W 32 KiB) copied by DMA into a two-stage LDS ring: right after the
// barrier that frees a slot, every wave issues 9 copies of the next stage, 5 of X and 4
// of W, then runs its 80 MFMAs on the current one.  Spreading the weight copies (HBM
// misses) over all waves keeps any one wave from queueing behind them; the two waves of
// a SIMD still finish a stage apart, the older one ahead.  Stages run on across
// blocks.  A range of ~9.3 groups ends in a short block of one or two groups: there the
// waves whose 128 columns are all past the end skip their MFMAs and the weight copies of
// absent rows are not issued (~23 % of the MFMAs were on such columns).  Rows beyond m
// re-read row m - 1 and are never stored; more than 320 rows take further passes.
constexpr int kLmMaxGrid = 256;  // persistent work-groups (one per CU)
constexpr int kLmRows = 320;
constexpr int kLmCols = 256;
constexpr int kLmWaves = 8;
constexpr int kLmSK = 64;
constexpr int kLmRing = 2;
constexpr int kLmXBytes = kLmRows * kLmSK * 2;   // 40 KiB
constexpr int kLmWBytes = kLmCols * kLmSK * 2;   // 32 KiB
constexpr int kLmStage = kLmXBytes + kLmWBytes;
constexpr int kLmInstr = kLmStage / 1024 / kLmWaves;  // DMA instructions per wave per stage (9)
static_assert(kLmStage % (1024 * kLmWaves) == 0, "stage split over waves");

struct LmStage {
  int m0, c0, ccols, k0;
};

// This wave's 9 copies of a stage: copy j moves 8 rows of 128 bytes (64 bf16) into LDS
// slot i = 8 j + wave, so copies 0..4 of every wave are X slots (i < 40) and 5..8 weight
// slots; row r keeps its 16-byte chunk c at position c ^ (r & 7).  A copy's source is a
// scalar base for the stage (X: k0; W: the block's first column and k0) plus a 32-bit
// lane offset that depends only on the pass's first row (X) or the block's width (W), so
// a stage's copies need no 64-bit arithmetic.
constexpr int kLmXCopies = kLmXBytes / 1024 / kLmWaves;  // 5
static_assert(kLmXBytes % (1024 * kLmWaves) == 0, "X slots split evenly over the waves");

struct LmCopies {
  uint32_t off[kLmInstr];
};

__device__ __forceinline__ void lm_offsets(const GemmParams& p, const LmStage& st, int wave, int lane,
                                           LmCopies& c) {
#pragma unroll
  for (int j = 0; j < kLmInstr; ++j) {
    const int i = j * kLmWaves + wave;
    if (j < kLmXCopies) {
      const int row = i * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ (row & 7);
      const int grow = min(st.m0 + row, p.m - 1);
      c.off[j] = (uint32_t)grow * (uint32_t)(p.ldx * 2) + (uint32_t)chunk * 16u;
    } else {
      const int wrow = (i - kLmXBytes / 1024) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ (wrow & 7);
      // a short block re-reads its last column
      c.off[j] = (uint32_t)min(wrow, st.ccols - 1) * (uint32_t)(p.k * 2) + (uint32_t)chunk * 16u;
    }
  }
}

__device__ __forceinline__ void lm_issue(const GemmParams& p, char* stage, const LmStage& st, const LmCopies& c,
                                         int wave) {
  const char* xsrc = uniform_ptr((const char*)p.x + st.k0 * 2);
  const char* wsrc = uniform_ptr((const char*)p.w + ((int64_t)st.c0 * p.k + st.k0) * 2);
#pragma unroll
  for (int j = 0; j < kLmInstr; ++j) {
    // weight slot j * 8 + wave - 40 holds rows (slot) 8 .. + 8 of the block: not copied when
    // they are all past a short block's end (those rows' MFMA outputs are never used)
    if (j >= kLmXCopies && (j * kLmWaves + wave - kLmXBytes / 1024) * 8 >= st.ccols) continue;
    uint32_t o = c.off[j];
    __asm__("" : "+v"(o));  // scalar base + 32-bit lane offset addressing
    lds_dma16((j < kLmXCopies ? xsrc : wsrc) + o, stage + (j * kLmWaves + wave) * 1024);
  }
}

__device__ __forceinline__ bf16x8 lm_frag(const char* base, int row, int chunk) {
  return __builtin_bit_cast(bf16x8, *(const u32x4*)(base + row * 128 + ((chunk ^ (row & 7)) * 16)));
}

// A stage's 80 MFMAs: two k-steps of 32 (lane group g holds k = 32 s + 8 g .. +8), the
// X fragment of token subtile mi + 1 read while the MFMAs of subtile mi run.
__device__ __forceinline__ void lm_mma(const char* stage, int mw, int nw, int lane, floatx4 (&acc)[5][8]) {
  const int r = lane & 15;
  const int g = lane >> 4;
  const char* xs = stage;
  const char* ws = stage + kLmXBytes;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bf16x8 b[8];
#pragma unroll
    for (int ns = 0; ns < 8; ++ns) b[ns] = lm_frag(ws, nw * 128 + ns * 16 + r, 4 * s + g);
    bf16x8 a = lm_frag(xs, mw * 80 + r, 4 * s + g);
#pragma unroll
    for (int mi = 0; mi < 5; ++mi) {
      bf16x8 an = a;
      if (mi < 4) an = lm_frag(xs, mw * 80 + (mi + 1) * 16 + r, 4 * s + g);
#pragma unroll
      for (int ns = 0; ns < 8; ++ns)
        acc[mi][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[ns], a, acc[mi][ns], 0, 0, 0);
      a = an;
    }
  }
}

// A bf16 pair (lo in bits 0..15) as two unsigned 16-bit codes in value order: positives
// 0x8000 + magnitude, negatives 0x8000 - magnitude, so -0 and +0 share 0x8000 (as
// torch.argmax treats them) and any finite value codes above 0.
__device__ __forceinline__ uint32_t bf16x2_order(uint32_t pair) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const uint32_t sgn = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, pair) >> (short)15);
  const uint32_t t = pair ^ ((sgn & 0x7FFF7FFFu) | 0x80008000u);
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, t) - __builtin_bit_cast(u16x2, sgn));
}

__global__ __launch_bounds__(kLmWaves * kWave) void lm_head_kernel(GemmParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int mw = wave & 3;
  const int nw = wave >> 2;
  const int r = lane & 15;
  const int g = lane >> 4;
  // this work-group's 64-column groups [grp0, grp1)
  const int groups = p.n / kArgmaxCols;
  const int grp0 = (int)((int64_t)groups * blockIdx.x / gridDim.x);
  const int grp1 = (int)((int64_t)groups * (blockIdx.x + 1) / gridDim.x);
  const int nblk = (grp1 - grp0 + 3) / 4;
  const int kt = p.k / kLmSK;
  const int mpass = (p.m + kLmRows - 1) / kLmRows;
  const int total = mpass * nblk * kt;  // stages, in order pass, block, k
  if (total == 0) return;
  // stages advance by counters (pass, block, k), so no stage needs a division
  auto make = [&](int pass, int bi, int t) {
    LmStage st;
    st.m0 = pass * kLmRows;
    st.c0 = (grp0 + 4 * bi) * kArgmaxCols;
    st.ccols = min(4, grp1 - grp0 - 4 * bi) * kArgmaxCols;
    st.k0 = t * kLmSK;
    return st;
  };
  int pass = 0, bi = 0, t = 0;
  // per token subtile: the best (value, index) key of row 16 mi + r over this wave's
  // columns of the pass so far; written once per pass as partial (row, 2 block + nw)
  // per token subtile: (order code << 16) | (0xFFFF - column within the range) of the best
  // value of row 16 mi + r over this lane's columns of the pass so far (0: none yet)
  uint32_t row_best[5] = {0, 0, 0, 0, 0};
  const int rc0 = grp0 * kArgmaxCols;
  const int tiles = 2 * (int)gridDim.x;

  floatx4 acc[5][8];
#pragma unroll
  for (int mi = 0; mi < 5; ++mi)
#pragma unroll
    for (int ns = 0; ns < 8; ++ns) acc[mi][ns] = floatx4{0.f, 0.f, 0.f, 0.f};

  LmStage cur = make(0, 0, 0);
  LmCopies copies;
  lm_offsets(p, cur, wave, lane, copies);
  int off_m0 = cur.m0, off_cols = cur.ccols;  // what the offsets were built for
  lm_issue(p, smem, cur, copies, wave);
  for (int u = 0; u < total; ++u) {
    wait_vmcnt<0>();                                   // this wave's copies of stage u
    asm volatile("s_barrier" ::: "memory");           // everyone's; stage u - 1 fully read
    const bool more = u + 1 < total;
    int npass = pass, nbi = bi, nt = t + 1;
    if (nt == kt) {
      nt = 0;
      if (++nbi == nblk) {
        nbi = 0;
        ++npass;
      }
    }
    const LmStage nst = more ? make(npass, nbi, nt) : cur;
    if (more && (nst.m0 != off_m0 || nst.ccols != off_cols)) {
      lm_offsets(p, nst, wave, lane, copies);
      off_m0 = nst.m0;
      off_cols = nst.ccols;
    }
    const int cur_cols = cur.ccols;
    if (more) lm_issue(p, smem + ((u + 1) & 1) * kLmStage, nst, copies, wave);
    if (nw * 128 < cur_cols) lm_mma(smem + (u & 1) * kLmStage, mw, nw, lane, acc);
    const bool block_done = t == kt - 1;
    const bool pass_done = block_done && (!more || npass != pass);
    const LmStage st = cur;
    cur = nst;
    pass = npass;
    bi = nbi;
    t = nt;
    if (!block_done) continue;

    // ---- block done: logits and argmax partials, then clear the accumulators ----
    // a lane's 32 values of a row are ranked by (order code << 16) | (31 - position),
    // position 4 ns + i in column order, then turned into a range column once per row
    const int ngrp = st.ccols / kArgmaxCols;
    const uint32_t col0 = (uint32_t)(st.c0 - rc0 + nw * 128 + 4 * g);
#pragma unroll
    for (int mi = 0; mi < 5; ++mi) {
      const int m = st.m0 + mw * 80 + mi * 16 + r;
      uint32_t best = 0;
#pragma unroll
      for (int q = 0; q < 2; ++q) {  // the wave's two 64-column groups
        const int grp = 2 * nw + q;
#pragma unroll
        for (int nq = 0; nq < 4; ++nq) {
          const int ns = 4 * q + nq;
          const int n = st.c0 + nw * 128 + ns * 16 + 4 * g;
          const floatx4 v = acc[mi][ns];
          const u32x2 bits = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          if (p.y != nullptr && m < p.m && grp < ngrp) *(u32x2*)(p.y + (int64_t)m * p.ldy + n) = bits;
          if (grp < ngrp) {
            const uint32_t o0 = bf16x2_order(bits[0]);
            const uint32_t o1 = bf16x2_order(bits[1]);
            const uint32_t rank = 31u - 4u * ns;
            best = max(best, (o0 << 16) | rank);
            best = max(best, (o0 & 0xFFFF0000u) | (rank - 1u));
            best = max(best, (o1 << 16) | (rank - 2u));
            best = max(best, (o1 & 0xFFFF0000u) | (rank - 3u));
          }
          acc[mi][ns] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
      }
      const uint32_t pos = 31u - (best & 31u);
      const uint32_t col = col0 + (pos >> 2) * 16u + (pos & 3u);
      if (best != 0) row_best[mi] = max(row_best[mi], (best & 0xFFFF0000u) | (0xFFFFu - col));
      if (pass_done) {
        uint32_t b2 = row_best[mi];
        b2 = max(b2, (uint32_t)__shfl_xor(b2, 16));
        b2 = max(b2, (uint32_t)__shfl_xor(b2, 32));
        if (p.argmax != nullptr && g == 0 && m < p.m) {
          const uint32_t n = (uint32_t)rc0 + 0xFFFFu - (b2 & 0xFFFFu);
          p.argmax[(int64_t)m * tiles + 2 * blockIdx.x + nw] =
              b2 == 0 ? 0 : ((uint64_t)(b2 >> 16) << 32) | (uint64_t)(0xFFFFFFFFu - n);
        }
        row_best[mi] = 0;
      }
    }
  }
}

// ---- LM head for at most 80 rows (a draft model's one-row-per-sequence decode, small
// verify batches) -------------------------------------------------------------------
// The 320-row kernel's time does not shrink with the rows: its eight waves split the
// rows four ways, so at m <= 80 two waves of one SIMD do all the MFMAs while the weights
// stream through the same two-stage ring.  Here wave c of a work-group owns columns
// 32 c .. +32 of each 256-column block against all 80 rows (5 x 2 subtiles), and a stage
// is X 10 KiB + W 32 KiB, so the ring holds three stages and the weight copies of a stage
// go out two stages ahead.  Work-group ranges, blocks, K stages, the chunk swizzle, the
// MFMA operand order and the argmax key are the 320-row kernel's: every logit is the same
// sum in the same order, hence the same bits, and so is every argmax partial.
constexpr int kLsRows = 80;
constexpr int kLsRing = 3;
constexpr int kLsXSlots = kLsRows * kLmSK * 2 / 1024;    // 10 copies of 8 rows
constexpr int kLsWSlots = kLmCols * kLmSK * 2 / 1024;    // 32
constexpr int kLsSlots = kLsXSlots + kLsWSlots;          // 42 per stage
constexpr int kLsStage = kLsSlots * 1024;
constexpr int kLsMaxCopies = (kLsSlots + kLmWaves - 1) / kLmWaves;  // 6 (waves 0, 1), else 5
static_assert(kLsRing * kLsStage <= 160 * 1024, "LDS");

// copy j of wave w fills stage slot s = 8 j + w (slots 0..9: X rows 8 s .., then W rows)
__device__ __forceinline__ int ls_copies(int wave) { return (kLsSlots - wave + kLmWaves - 1) / kLmWaves; }

__global__ __launch_bounds__(kLmWaves * kWave) void lm_head_small_kernel(GemmParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int groups = p.n / kArgmaxCols;
  const int grp0 = (int)((int64_t)groups * blockIdx.x / gridDim.x);
  const int grp1 = (int)((int64_t)groups * (blockIdx.x + 1) / gridDim.x);
  const int nblk = (grp1 - grp0 + 3) / 4;
  const int kt = p.k / kLmSK;
  const int total = nblk * kt;  // stages, in order block, k
  if (total == 0) return;
  const int rc0 = grp0 * kArgmaxCols;
  const int tiles = 2 * (int)gridDim.x;
  const int ncp = ls_copies(wave);

  // per copy: the 32-bit lane offset from the stage's scalar base (X: row and chunk; W:
  // column row within the block and chunk, a short block re-reading its last column)
  auto offset = [&](int j, int ccols) -> uint32_t {
    const int s = j * kLmWaves + wave;
    if (s < kLsXSlots) {
      const int row = s * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ (row & 7);
      return (uint32_t)min(row, p.m - 1) * (uint32_t)(p.ldx * 2) + (uint32_t)chunk * 16u;
    }
    const int wrow = (s - kLsXSlots) * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (wrow & 7);
    return (uint32_t)min(wrow, ccols - 1) * (uint32_t)(p.k * 2) + (uint32_t)chunk * 16u;
  };
  auto issue = [&](int u) {
    const int bi = u / kt, t = u % kt;
    const int c0 = (grp0 + 4 * bi) * kArgmaxCols;
    const int ccols = min(4, grp1 - grp0 - 4 * bi) * kArgmaxCols;
    const int k0 = t * kLmSK;
    char* stage = smem + (u % kLsRing) * kLsStage;
    const char* xsrc = uniform_ptr((const char*)p.x + k0 * 2);
    const char* wsrc = uniform_ptr((const char*)p.w + ((int64_t)c0 * p.k + k0) * 2);
#pragma unroll
    for (int j = 0; j < kLsMaxCopies; ++j) {
      if (j >= ncp) break;
      const int s = j * kLmWaves + wave;
      uint32_t o = offset(j, ccols);
      __asm__("" : "+v"(o));  // scalar base + 32-bit lane offset addressing
      lds_dma16((s < kLsXSlots ? xsrc : wsrc) + o, stage + s * 1024);
    }
  };

  floatx4 acc[5][2];
#pragma unroll
  for (int mi = 0; mi < 5; ++mi) acc[mi][0] = acc[mi][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  uint32_t row_best[5] = {0, 0, 0, 0, 0};

  issue(0);
  if (total > 1) issue(1);
  for (int u = 0; u < total; ++u) {
    // this wave's copies of stage u have landed once at most stage u + 1's are in flight
    if (u + 1 < total) {
      wait_pending<1, kLsMaxCopies>(ncp);
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("s_barrier" ::: "memory");  // everyone's stage u; stage u - 1 fully read
    if (u + 2 < total) issue(u + 2);
    const int bi = u / kt, t = u % kt;
    const int c0 = (grp0 + 4 * bi) * kArgmaxCols;
    const int ccols = min(4, grp1 - grp0 - 4 * bi) * kArgmaxCols;
    const bool live = wave * 32 < ccols;  // a short block's waves past its end skip the MFMAs
    if (live) {
      const char* xs = smem + (u % kLsRing) * kLsStage;
      const char* ws = xs + kLsXSlots * 1024;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bf16x8 b[2];
#pragma unroll
        for (int ns = 0; ns < 2; ++ns) b[ns] = lm_frag(ws, wave * 32 + ns * 16 + r, 4 * s + g);
#pragma unroll
        for (int mi = 0; mi < 5; ++mi) {
          const bf16x8 a = lm_frag(xs, mi * 16 + r, 4 * s + g);
#pragma unroll
          for (int ns = 0; ns < 2; ++ns)
            acc[mi][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[ns], a, acc[mi][ns], 0, 0, 0);
        }
      }
    }
    if (t != kt - 1) continue;

    // ---- block done: logits, this lane's best of its 8 values per row, clear ----
    const uint32_t col0 = (uint32_t)(c0 - rc0 + wave * 32 + 4 * g);
#pragma unroll
    for (int mi = 0; mi < 5; ++mi) {
      const int m = mi * 16 + r;
      uint32_t best = 0;
#pragma unroll
      for (int ns = 0; ns < 2; ++ns) {
        const floatx4 v = acc[mi][ns];
        const u32x2 bits = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        if (p.y != nullptr && m < p.m && live)
          *(u32x2*)(p.y + (int64_t)m * p.ldy + c0 + wave * 32 + ns * 16 + 4 * g) = bits;
        if (live) {
          const uint32_t o0 = bf16x2_order(bits[0]);
          const uint32_t o1 = bf16x2_order(bits[1]);
          const uint32_t rank = 7u - 4u * ns;
          best = max(best, (o0 << 16) | rank);
          best = max(best, (o0 & 0xFFFF0000u) | (rank - 1u));
          best = max(best, (o1 << 16) | (rank - 2u));
          best = max(best, (o1 & 0xFFFF0000u) | (rank - 3u));
        }
        acc[mi][ns] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
      const uint32_t pos = 7u - (best & 7u);
      const uint32_t col = col0 + (pos >> 2) * 16u + (pos & 3u);
      if (best != 0) row_best[mi] = max(row_best[mi], (best & 0xFFFF0000u) | (0xFFFFu - col));
    }
  }

  // ---- the range's argmax partials: per row, the best of the four waves of each
  // 128-column half (waves 0..3, 4..7), as the 320-row kernel's waves nw = 0, 1 keep them
  uint32_t* s_best = (uint32_t*)smem;  // [wave][80 rows]
  __syncthreads();                     // every wave is past its last stage
#pragma unroll
  for (int mi = 0; mi < 5; ++mi) {
    uint32_t b2 = row_best[mi];
    b2 = max(b2, (uint32_t)__shfl_xor(b2, 16));
    b2 = max(b2, (uint32_t)__shfl_xor(b2, 32));
    if (g == 0) s_best[wave * kLsRows + mi * 16 + r] = b2;
  }
  __syncthreads();
  if (p.argmax != nullptr && (wave & 3) == 0) {
    const int half = wave >> 2;
    for (int m = lane; m < p.m; m += kWave) {
      uint32_t b2 = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) b2 = max(b2, s_best[(half * 4 + w) * kLsRows + m]);
      const uint32_t n = (uint32_t)rc0 + 0xFFFFu - (b2 & 0xFFFFu);
      p.argmax[(int64_t)m * tiles + 2 * blockIdx.x + half] =
          b2 == 0 ? 0 : ((uint64_t)(b2 >> 16) << 32) | (uint64_t)(0xFFFFFFFFu - n);
    }
  }
}

int launch_lm_head(GemmParams p, hipStream_t stream) {
  const int groups = p.n / kArgmaxCols;
  const int grid = groups < kLmMaxGrid ? groups : kLmMaxGrid;
  if (p.m <= kLsRows) {
    static const hipError_t attr_small = hipFuncSetAttribute(
        (const void*)lm_head_small_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kLsRing * kLsStage);
    if (attr_small != hipSuccess) {
      set_error("lm_head: cannot reserve %d bytes of LDS: %s", kLsRing * kLsStage, hipGetErrorString(attr_small));
      return NE_ELAUNCH;
    }
    hipLaunchKernelGGL(lm_head_small_kernel, dim3((unsigned)grid), dim3(kLmWaves * kWave), kLsRing * kLsStage,
                       stream, p);
    return check_launch("lm_head");
  }
  static const hipError_t attr = hipFuncSetAttribute(
      (const void*)lm_head_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kLmRing * kLmStage);
  if (attr != hipSuccess) {
    set_error("lm_head: cannot reserve %d bytes of LDS: %s", kLmRing * kLmStage, hipGetErrorString(attr));
    return NE_ELAUNCH;
  }
  hipLaunchKernelGGL(lm_head_kernel, dim3((unsigned)grid), dim3(kLmWaves * kWave), kLmRing * kLmStage, stream, p);
  return check_launch("lm_head");
}

}  // namespace

}  // namespace ne

using namespace ne;

namespace {

int w8a16_common(const void* x, int64_t ldx, const int8_t* w, const void* scale, int32_t scale_dtype,
                 int32_t m, int32_t n, int32_t k, void* y, int64_t ldy, int32_t epilogue,
                 int32_t splits, float* partial, void* stream) {
  GemmParams p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = w;
  p.scale = scale;
  p.m = m;
  p.n = n;
  p.k = k;
  p.y = (uint16_t*)y;
  p.ldy = ldy;
  hipStream_t s = (hipStream_t)stream;
  switch (scale_dtype) {
    case NE_DTYPE_BF16:
      return dispatch_w8a16<NE_DTYPE_BF16>(p, epilogue, splits, partial, s);
    case NE_DTYPE_FP16:
      return dispatch_w8a16<NE_DTYPE_FP16>(p, epilogue, splits, partial, s);
    case NE_DTYPE_FP32:
      return dispatch_w8a16<NE_DTYPE_FP32>(p, epilogue, splits, partial, s);
    default:
      set_error("scale_dtype must be bf16, fp16 or fp32");
      return NE_EINVAL;
  }
}

}  // namespace

extern "C" int ne_w8a16_gemm(const void* x, int64_t ldx, const int8_t* w, const void* scale,
                             int32_t scale_dtype, int32_t m, int32_t n, int32_t k, void* y,
                             int64_t ldy, int32_t epilogue, void* stream) {
  NE_CHECK_ARG(m >= 0 && n > 0 && k > 0, "bad gemm shape m=%d n=%d k=%d", m, n, k);
  if (m == 0) return NE_OK;
  NE_CHECK_ARG(x && w && scale && y, "null pointer argument");
  NE_CHECK_ARG(epilogue == NE_EPILOGUE_STORE || epilogue == NE_EPILOGUE_SWIGLU,
               "unknown epilogue %d", epilogue);
  NE_CHECK_SUPPORTED(k % 128 == 0, "k must be a multiple of 128 (got %d)", k);
  NE_CHECK_SUPPORTED(n % 64 == 0, "n must be a multiple of 64 (got %d)", n);
  NE_CHECK_ARG(ldx >= k && ldx % 8 == 0, "ldx must be >= k and a multiple of 8");
  NE_CHECK_SUPPORTED((int64_t)m * ldx < kMaxXElems, "x spans more than 4 GiB (m=%d, ldx=%lld)", m, (long long)ldx);
  NE_CHECK_ARG(ldy >= (epilogue == NE_EPILOGUE_SWIGLU ? n / 2 : n) && ldy % 4 == 0,
               "ldy too small or not a multiple of 4");
  NE_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)y % 8) == 0,
               "x and w must be 16-byte aligned, y 8-byte aligned");
  return w8a16_common(x, ldx, w, scale, scale_dtype, m, n, k, y, ldy, epilogue, 1, nullptr, stream);
}

extern "C" int ne_w8a16_gemm_splitk(const void* x, int64_t ldx, const int8_t* w, const void* scale,
                                    int32_t scale_dtype, int32_t m, int32_t n, int32_t k,
                                    int32_t splits, float* partials, void* stream) {
  NE_CHECK_ARG(m >= 0 && n > 0 && k > 0, "bad gemm shape m=%d n=%d k=%d", m, n, k);
  if (m == 0) return NE_OK;
  NE_CHECK_ARG(x && w && scale && partials, "null pointer argument");
  NE_CHECK_ARG(splits >= 1 && splits <= 64, "splits must be in [1, 64] (got %d)", splits);
  NE_CHECK_SUPPORTED(k % (128 * splits) == 0, "k must be a multiple of 128 * splits (k=%d, splits=%d)",
                     k, splits);
  NE_CHECK_SUPPORTED(n % 64 == 0, "n must be a multiple of 64 (got %d)", n);
  NE_CHECK_ARG(ldx >= k && ldx % 8 == 0, "ldx must be >= k and a multiple of 8");
  NE_CHECK_SUPPORTED((int64_t)m * ldx < kMaxXElems, "x spans more than 4 GiB (m=%d, ldx=%lld)", m, (long long)ldx);
  NE_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)partials % 16) == 0,
               "x, w and partials must be 16-byte aligned");
  return w8a16_common(x, ldx, w, scale, scale_dtype, m, n, k, nullptr, 0, NE_EPILOGUE_STORE, splits,
                      partials, stream);
}

extern "C" int ne_w8a16_qkv_norm_rope_kv(
    const void* x, int64_t ldx, const int8_t* w, const void* scale, int32_t scale_dtype, int32_t m,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t k, const void* q_norm_w, const void* k_norm_w,
    float eps, const int32_t* positions, const void* rope, int32_t rope_positions,
    const int32_t* slot_mapping, int32_t kv_dtype, void* k_cache, void* v_cache, void* k_scale,
    void* v_scale, int32_t kv_scale_dtype, void* q_out, void* stream) {
  NE_CHECK_ARG(m >= 0 && num_q_heads > 0 && num_kv_heads > 0 && k > 0, "bad shape");
  if (m == 0) return NE_OK;
  NE_CHECK_ARG(x && w && scale && q_norm_w && k_norm_w && positions && rope && slot_mapping && k_cache &&
                   v_cache && q_out,
               "null pointer argument");
  NE_CHECK_ARG(rope_positions > 0, "rope_positions must be > 0");
  NE_CHECK_SUPPORTED(k % 128 == 0, "k must be a multiple of 128 (got %d)", k);
  NE_CHECK_ARG(ldx >= k && ldx % 8 == 0, "ldx must be >= k and a multiple of 8");
  NE_CHECK_SUPPORTED((int64_t)m * ldx < kMaxXElems, "x spans more than 4 GiB (m=%d, ldx=%lld)", m, (long long)ldx);
  NE_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0, "x and w must be 16-byte aligned");
  int kv_mode = 0;
  if (kv_dtype == NE_DTYPE_BF16) {
    kv_mode = 1;
  } else if (kv_dtype == NE_DTYPE_INT8) {
    NE_CHECK_ARG(k_scale && v_scale, "an int8 cache needs k_scale and v_scale");
    NE_CHECK_SUPPORTED(kv_scale_dtype == NE_DTYPE_BF16 || kv_scale_dtype == NE_DTYPE_FP16,
                       "fused KV write supports bf16 or fp16 scales");
    kv_mode = kv_scale_dtype == NE_DTYPE_BF16 ? 2 : 3;
  } else {
    set_error("kv_dtype must be int8 or bf16");
    return NE_EINVAL;
  }
  GemmParams p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = w;
  p.scale = scale;
  p.m = m;
  p.n = (num_q_heads + 2 * num_kv_heads) * 128;
  p.k = k;
  const QkvRopeArgs qa{num_q_heads, num_kv_heads, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w,
                       eps, positions, (const uint16_t*)rope, rope_positions, slot_mapping,
                       k_cache, v_cache, k_scale, v_scale, (uint16_t*)q_out};
  hipStream_t s = (hipStream_t)stream;
  switch (scale_dtype) {
    case NE_DTYPE_BF16: return dispatch_qkv_fused<NE_DTYPE_BF16>(p, qa, kv_mode, s);
    case NE_DTYPE_FP16: return dispatch_qkv_fused<NE_DTYPE_FP16>(p, qa, kv_mode, s);
    case NE_DTYPE_FP32: return dispatch_qkv_fused<NE_DTYPE_FP32>(p, qa, kv_mode, s);
    default:
      set_error("scale_dtype must be bf16, fp16 or fp32");
      return NE_EINVAL;
  }
}

extern "C" int32_t ne_lm_head_num_tiles(int32_t n) {
  return n > 0 ? 2 * min(n / kArgmaxCols, kLmMaxGrid) : 0;  // two waves' halves per work-group
}

extern "C" int ne_lm_head(const void* x, int64_t ldx, const void* w, int32_t m, int32_t n,
                          int32_t k, void* logits, int64_t ld_logits, uint64_t* argmax_partials,
                          void* stream) {
  NE_CHECK_ARG(m >= 0 && n > 0 && k > 0, "bad lm head shape m=%d n=%d k=%d", m, n, k);
  if (m == 0) return NE_OK;
  NE_CHECK_ARG(x && w, "null pointer argument");
  NE_CHECK_ARG(logits || argmax_partials, "lm head needs logits and/or argmax_partials");
  NE_CHECK_SUPPORTED(k % 128 == 0, "k must be a multiple of 128 (got %d)", k);
  NE_CHECK_SUPPORTED(n % 128 == 0, "vocab must be a multiple of 128 (got %d)", n);
  // argmax keys hold a column within a work-group's range in 16 bits
  NE_CHECK_SUPPORTED(n <= (1 << 24), "vocab above 2^24 (got %d)", n);
  NE_CHECK_ARG(ldx >= k && ldx % 8 == 0, "ldx must be >= k and a multiple of 8");
  NE_CHECK_ARG(!logits || (ld_logits >= n && ld_logits % 4 == 0), "bad ld_logits");
  NE_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 &&
                   ((uintptr_t)logits % 8) == 0,
               "x and w must be 16-byte aligned, logits 8-byte aligned");
  // X copies address rows with 32-bit byte offsets, weight rows of a block likewise
  NE_CHECK_SUPPORTED((int64_t)m * ldx < kMaxXElems, "x spans more than 4 GiB (m=%d, ldx=%lld)", m, (long long)ldx);
  NE_CHECK_SUPPORTED((int64_t)kLmCols * k * 2 < (int64_t(1) << 32), "k too large for the LM head (k=%d)", k);
  GemmParams p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = w;
  p.m = m;
  p.n = n;
  p.k = k;
  p.y = (uint16_t*)logits;
  p.ldy = ld_logits;
  p.argmax = argmax_partials;
  hipStream_t s = (hipStream_t)stream;
  return launch_lm_head(p, s);
}
