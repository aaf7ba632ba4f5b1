// W8A16 projection GEMMs and the bf16 LM-head GEMM for gfx950.
//
// Replaces Int8Linear.forward (ne/models/int8_quantization.py:55-57), which
// materialises bf16(int8 * scale) for the whole weight before F.linear, and the
// tied-embedding LM head (ne/models/qwen3.py:197-203).
//
// Each 16x16 MFMA tile computes D = W . X^T (weight rows x token rows) with
// v_mfma_f32_16x16x32_bf16, so a lane ends up holding four consecutive output
// columns of one token row (8-byte stores) and the weight operand can be loaded
// straight from global memory into registers:
//   lane l, weight subtile: weight row l % 16, k = (l/16)*BK/4 .. +BK/4
//   lane l, token subtile : token row  l % 16, same k range (read from LDS)
// int8 weights become bf16 in registers (one SDWA convert per byte; exact) and
// the per-output-row scale is applied to the fp32 accumulator.  The token tile
// X[BM x BK] is staged through LDS (double buffered) and shared by the 4 waves
// of a work-group; wave w owns NW weight subtiles (16 rows each) and all BM
// token rows.  Work-group ids are mapped so that the M blocks of one weight
// tile run on the same XCD (shared L2).
#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kThreads = 256;
constexpr int kGemmWaves = 4;

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

// per-lane weight registers for one BK slice of one 16-row subtile
template <int BK, bool WINT8>
struct WRegs {
  static constexpr int kBytes = WINT8 ? BK / 4 : BK / 2;  // 16/8 B int8, 32/16 B bf16
  static constexpr int kVec = (kBytes + 15) / 16;
  u32x4 v[kVec];
};

template <int BK, bool WINT8>
__device__ __forceinline__ void load_w(const GemmParams& p, int row, int k0, int lane,
                                       WRegs<BK, WINT8>& R) {
  const int kk = k0 + (lane >> 4) * (BK / 4);
  if constexpr (WINT8) {
    const int8_t* src = (const int8_t*)p.w + (int64_t)row * p.k + kk;
    if constexpr (BK == 64) {
      R.v[0] = *(const u32x4*)src;
    } else {
      const u32x2 t = *(const u32x2*)src;
      R.v[0] = u32x4{t[0], t[1], 0, 0};
    }
  } else {
    const u32x4* src = (const u32x4*)((const uint16_t*)p.w + (int64_t)row * p.k + kk);
#pragma unroll
    for (int i = 0; i < WRegs<BK, WINT8>::kVec; ++i) R.v[i] = src[i];
  }
}

template <int BK, bool WINT8>
__device__ __forceinline__ bf16x8 w_operand(const WRegs<BK, WINT8>& R, int s) {
  if constexpr (WINT8) {
    return int8x8_to_bf16x8(R.v[0][2 * s], R.v[0][2 * s + 1]);
  } else {
    return __builtin_bit_cast(bf16x8, R.v[s]);
  }
}

template <int SDT>
__device__ __forceinline__ float scale_at(const void* s, int64_t i) {
  if constexpr (SDT < 0) {
    return 1.f;
  } else {
    return load_scale<SDT>(s, i);
  }
}

// EPI: 0 store, 1 swiglu, 2 lm head (optional store + argmax partials)
template <int MW, int NW, int BK, bool WINT8, int SDT, int EPI>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams p) {
  constexpr int BM = MW * 16;
  constexpr int BN = kGemmWaves * NW * 16;
  constexpr int KS = BK / 32;        // MFMA k-steps per BK slice
  constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (bank spread)
  constexpr int XV = BM * BK / 8;     // 16-byte vectors per X tile
  constexpr int XV_PER_T = (XV + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) uint16_t s_x[2][BM * LDS_STRIDE];
  __shared__ uint64_t s_best[kGemmWaves][BM];

  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int jj = bid / kNumXcd;
  const int tm = jj % p.tiles_m;
  const int tn = (jj / p.tiles_m) * kNumXcd + xcd;
  if (tn >= p.tiles_n) return;
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wrow0 = n0 + wave * NW * 16;  // first weight row of this wave

  floatx4 acc[MW][NW];
#pragma unroll
  for (int mi = 0; mi < MW; ++mi)
#pragma unroll
    for (int ni = 0; ni < NW; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto load_x = [&](int k0, u32x4(&xr)[XV_PER_T]) {
#pragma unroll
    for (int i = 0; i < XV_PER_T; ++i) {
      const int idx = tid + i * kThreads;
      const int row = idx / (BK / 8);
      const int c8 = idx % (BK / 8);
      u32x4 v = {0, 0, 0, 0};
      if (idx < XV && m0 + row < p.m)
        v = *(const u32x4*)(p.x + (int64_t)(m0 + row) * p.ldx + k0 + c8 * 8);
      xr[i] = v;
    }
  };
  auto store_x = [&](int buf, const u32x4(&xr)[XV_PER_T]) {
#pragma unroll
    for (int i = 0; i < XV_PER_T; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < XV) {
        const int row = idx / (BK / 8);
        const int c8 = idx % (BK / 8);
        *(u32x4*)&s_x[buf][row * LDS_STRIDE + c8 * 8] = xr[i];
      }
    }
  };

  const int n_k = p.k / BK;
  u32x4 xr[XV_PER_T];
  WRegs<BK, WINT8> wc[NW], wn[NW];
  load_x(0, xr);
#pragma unroll
  for (int ni = 0; ni < NW; ++ni) load_w<BK, WINT8>(p, wrow0 + ni * 16 + r, 0, lane, wc[ni]);
  store_x(0, xr);
  __syncthreads();

  for (int kt = 0; kt < n_k; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < n_k;
    if (more) {
      load_x((kt + 1) * BK, xr);
#pragma unroll
      for (int ni = 0; ni < NW; ++ni)
        load_w<BK, WINT8>(p, wrow0 + ni * 16 + r, (kt + 1) * BK, lane, wn[ni]);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 a[NW];
#pragma unroll
      for (int ni = 0; ni < NW; ++ni) a[ni] = w_operand<BK, WINT8>(wc[ni], s);
#pragma unroll
      for (int mi = 0; mi < MW; ++mi) {
        const bf16x8 b = __builtin_bit_cast(
            bf16x8, *(const u32x4*)&s_x[buf][(mi * 16 + r) * LDS_STRIDE + g * (BK / 4) + s * 8]);
#pragma unroll
        for (int ni = 0; ni < NW; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[ni], b, acc[mi][ni], 0, 0, 0);
      }
    }
    if (more) store_x(buf ^ 1, xr);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int ni = 0; ni < NW; ++ni) wc[ni] = wn[ni];
    }
  }

  // ---- epilogue: lane holds D[n = 4g + i][m = r] of every (mi, ni) tile ----
  if constexpr (EPI == 0) {
#pragma unroll
    for (int ni = 0; ni < NW; ++ni) {
      const int n = wrow0 + ni * 16 + 4 * g;
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[i] = scale_at<SDT>(p.scale, n + i);
#pragma unroll
      for (int mi = 0; mi < MW; ++mi) {
        const int m = m0 + mi * 16 + r;
        if (m < p.m) {
          const floatx4 v = acc[mi][ni];
          const u32x2 bits = {pack_bf16x2(v[0] * sc[0], v[1] * sc[1]),
                              pack_bf16x2(v[2] * sc[2], v[3] * sc[3])};
          *(u32x2*)(p.y + (int64_t)m * p.ldy + n) = bits;
        }
      }
    }
  } else if constexpr (EPI == 1) {
    static_assert(NW % 2 == 0, "swiglu pairs gate/up subtiles");
#pragma unroll
    for (int q = 0; q < NW / 2; ++q) {
      const int ng = wrow0 + 2 * q * 16 + 4 * g;  // gate rows; up rows are +16
      const int ncol = (wrow0 + 2 * q * 16) / 2 + 4 * g;
      float sg[4], su[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sg[i] = scale_at<SDT>(p.scale, ng + i);
        su[i] = scale_at<SDT>(p.scale, ng + 16 + i);
      }
#pragma unroll
      for (int mi = 0; mi < MW; ++mi) {
        const int m = m0 + mi * 16 + r;
        if (m < p.m) {
          float out[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gate = bf16_round(acc[mi][2 * q][i] * sg[i]);
            const float up = bf16_round(acc[mi][2 * q + 1][i] * su[i]);
            const float silu = bf16_round(gate / (1.f + __expf(-gate)));
            out[i] = silu * up;
          }
          const u32x2 bits = {pack_bf16x2(out[0], out[1]), pack_bf16x2(out[2], out[3])};
          *(u32x2*)(p.y + (int64_t)m * p.ldy + ncol) = bits;
        }
      }
    }
  } else {
    // LM head: optional bf16 logits and per-(row, tile) argmax of bf16 logits
#pragma unroll
    for (int mi = 0; mi < MW; ++mi) {
      const int m = m0 + mi * 16 + r;
      uint64_t best = 0;
#pragma unroll
      for (int ni = 0; ni < NW; ++ni) {
        const int n = wrow0 + ni * 16 + 4 * g;
        const floatx4 v = acc[mi][ni];
        const u32x2 bits = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        if (p.y != nullptr && m < p.m) *(u32x2*)(p.y + (int64_t)m * p.ldy + n) = bits;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float rv = bf16_to_f32((uint16_t)(bits[i >> 1] >> (16 * (i & 1))));
          best = max_u64(best, argmax_key(rv, (uint32_t)(n + i)));
        }
      }
      best = max_u64(best, shfl_xor_u64(best, 16));
      best = max_u64(best, shfl_xor_u64(best, 32));
      if (g == 0) s_best[wave][mi * 16 + r] = best;
    }
    if (p.argmax != nullptr) {
      __syncthreads();
      for (int row = tid; row < BM; row += kThreads) {
        const int m = m0 + row;
        if (m < p.m) {
          uint64_t b = s_best[0][row];
#pragma unroll
          for (int w = 1; w < kGemmWaves; ++w) b = max_u64(b, s_best[w][row]);
          p.argmax[(int64_t)m * p.tiles_n + tn] = b;
        }
      }
    }
  }
}

template <int MW, int NW, int BK, bool WINT8, int SDT, int EPI>
int launch_gemm(GemmParams p, hipStream_t stream, const char* name) {
  constexpr int BM = MW * 16;
  constexpr int BN = kGemmWaves * NW * 16;
  p.tiles_m = ceil_div(p.m, BM);
  p.tiles_n = p.n / BN;
  const int tiles_n_padded = ceil_div(p.tiles_n, kNumXcd) * kNumXcd;
  const dim3 grid((unsigned)(p.tiles_m * tiles_n_padded));
  hipLaunchKernelGGL((gemm_kernel<MW, NW, BK, WINT8, SDT, EPI>), grid, dim3(kThreads), 0, stream,
                     p);
  return check_launch(name);
}

template <int SDT>
int dispatch_w8a16(GemmParams p, int epilogue, hipStream_t s) {
  if (epilogue == NE_EPILOGUE_SWIGLU) {
    if (p.m <= 32) return launch_gemm<2, 2, 64, true, SDT, 1>(p, s, "w8a16_swiglu");
    return launch_gemm<4, 2, 64, true, SDT, 1>(p, s, "w8a16_swiglu");
  }
  if (p.m <= 32) return launch_gemm<2, 1, 64, true, SDT, 0>(p, s, "w8a16_gemm");
  return launch_gemm<4, 1, 64, true, SDT, 0>(p, s, "w8a16_gemm");
}

constexpr int kLmHeadBN = kGemmWaves * 16;

}  // namespace

}  // namespace ne

using namespace ne;

extern "C" int ne_w8a16_gemm(const void* x, int64_t ldx, const int8_t* w, const void* scale,
                             int32_t scale_dtype, int32_t m, int32_t n, int32_t k, void* y,
                             int64_t ldy, int32_t epilogue, void* stream) {
  NE_CHECK_ARG(m >= 0 && n > 0 && k > 0, "bad gemm shape m=%d n=%d k=%d", m, n, k);
  if (m == 0) return NE_OK;
  NE_CHECK_ARG(x && w && scale && y, "null pointer argument");
  NE_CHECK_ARG(epilogue == NE_EPILOGUE_STORE || epilogue == NE_EPILOGUE_SWIGLU,
               "unknown epilogue %d", epilogue);
  NE_CHECK_SUPPORTED(k % 64 == 0, "k must be a multiple of 64 (got %d)", k);
  const int bn = (epilogue == NE_EPILOGUE_SWIGLU) ? 128 : 64;
  NE_CHECK_SUPPORTED(n % bn == 0, "n must be a multiple of %d (got %d)", bn, n);
  NE_CHECK_ARG(ldx >= k && ldx % 8 == 0, "ldx must be >= k and a multiple of 8");
  NE_CHECK_ARG(ldy >= (epilogue == NE_EPILOGUE_SWIGLU ? n / 2 : n) && ldy % 4 == 0,
               "ldy too small or not a multiple of 4");
  NE_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)y % 8) == 0,
               "x and w must be 16-byte aligned, y 8-byte aligned");
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
      return dispatch_w8a16<NE_DTYPE_BF16>(p, epilogue, s);
    case NE_DTYPE_FP16:
      return dispatch_w8a16<NE_DTYPE_FP16>(p, epilogue, s);
    case NE_DTYPE_FP32:
      return dispatch_w8a16<NE_DTYPE_FP32>(p, epilogue, s);
    default:
      set_error("scale_dtype must be bf16, fp16 or fp32");
      return NE_EINVAL;
  }
}

extern "C" int32_t ne_lm_head_num_tiles(int32_t n) { return n > 0 ? n / kLmHeadBN : 0; }

extern "C" int ne_lm_head(const void* x, int64_t ldx, const void* w, int32_t m, int32_t n,
                          int32_t k, void* logits, int64_t ld_logits, uint64_t* argmax_partials,
                          void* stream) {
  NE_CHECK_ARG(m >= 0 && n > 0 && k > 0, "bad lm head shape m=%d n=%d k=%d", m, n, k);
  if (m == 0) return NE_OK;
  NE_CHECK_ARG(x && w, "null pointer argument");
  NE_CHECK_ARG(logits || argmax_partials, "lm head needs logits and/or argmax_partials");
  NE_CHECK_SUPPORTED(k % 32 == 0, "k must be a multiple of 32 (got %d)", k);
  NE_CHECK_SUPPORTED(n % kLmHeadBN == 0, "vocab must be a multiple of %d (got %d)", kLmHeadBN, n);
  NE_CHECK_ARG(ldx >= k && ldx % 8 == 0, "ldx must be >= k and a multiple of 8");
  NE_CHECK_ARG(!logits || (ld_logits >= n && ld_logits % 4 == 0), "bad ld_logits");
  NE_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 &&
                   ((uintptr_t)logits % 8) == 0,
               "x and w must be 16-byte aligned, logits 8-byte aligned");
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
  if (m <= 64) return launch_gemm<4, 1, 32, false, -1, 2>(p, s, "lm_head");
  if (m <= 128) return launch_gemm<8, 1, 32, false, -1, 2>(p, s, "lm_head");
  return launch_gemm<20, 1, 32, false, -1, 2>(p, s, "lm_head");
}
