// Fused acceptance for speculative verify on gfx950: greedy match or
// rejection sampling, correction/bonus token, KV-count rollback and history
// append, one 256-thread work-group per sequence.
//
// Restates verify_proposal (ne/engine/speculative/verifier.py:27-60) and
// compute_token_probabilities / apply_top_p (ne/engine/sampling.py:21-38); the
// rollback is num_cached = len_before + kept
// (ne/engine/speculative/speculative_generator.py:78-83).  Each sequence has its
// own temperature and top-p, so greedy and sampled requests share one call.
//
// Greedy (temperature 0, ne/engine/sampling.py:32-34): target token of a row is
// the argmax of its bf16 logits, first index on ties (torch.argmax order).
//
// Sampled (temperature T > 0).  The reference draws with torch.rand /
// torch.multinomial, which no other implementation reproduces; this library fixes
// explicit procedures instead, shared bit for bit with the CPU oracle.
//
// One-hot guesses (n-gram, and the draft model's own draws): the integer-mass
// contract.  Every token's weight is an integer that depends only on its bf16
// order key k (larger logit, larger key; -0 as +0), so sums in any order are exact:
//   invT = 1 / T (fp32 division); kmax = the row's largest key; mx = val(kmax) * invT
//   E(k) = (uint32)(exp3(val(k) * invT - mx) * 2^31), truncated (E(kmax) = 2^31; tokens
//          more than ~21.5 T below the largest logit weigh 0); exp3 = Cephes' Cody-Waite
//          reduction and degree-5 polynomial with every step one fused multiply-add,
//          0 below -86
//   cnt(k) = tokens of key k; Z = sum_k cnt(k) E(k)
//   top-p (P < 1): thr = max(1, (uint64)((double)Z * (double)P)); M(v) = sum_{k > v}
//          cnt(k) E(k); tau = the smallest v with M(v) < thr; m = min(cnt(tau),
//          ceil((thr - M(tau)) / E(tau))); kept: key > tau, or key == tau and fewer than m
//          tokens of key tau precede it; K = M(tau) + m E(tau).  P >= 1 keeps all, K = Z.
//   guess g of row i (U_i = the uniform's 24-bit integer): kept iff w_g >= K or
//          (w_g > 0 and U_i * K < w_g * 2^24), w_g = E(key_g) if g is kept, else 0 (also
//          for a guess outside the vocabulary)
//   draw (a rejected row: its guess removed; the bonus row: nothing removed): the kept
//          tokens in order of key (descending) then index (ascending), the guess removed
//          unless that leaves no weight; R = their weight; t = floor(U * R / 2^24); the
//          token is the first whose running weight exceeds t.
// accept_rows_kernel decides every sampled row in its own work-group (histogram of the
// row's keys, then key-space sums and one compare-only pass to place a draw); the
// finish keeps guesses up to the first row that drew.
//
// With draft rows (a draft model's distribution per guess) the earlier fp32 contract
// applies:
//   z_j  = fp32(logit_j) / T                  (IEEE fp32 division)
//   e_j  = cephes_exp(z_j - max_j z_j)        (Cephes expf, Moshier; 0 below -86)
//   chunked total of a row vector w: S_c = sequential fp32 sum of w_j over chunk
//          c = [c*CH, min((c+1)*CH, V)), CH = ceil(V / 256), c = 0..255; total =
//          sequential sum of S_0..S_255.  Z = chunked total of e.
//   top-p (top_p < 1): tokens rank by bf16 logit (larger first, -0 as +0), ties by
//          index.  M(v) = chunked total of e_j over tokens whose 16-bit key exceeds
//          v; thr = top_p * Z; tau = smallest key v with M(v) < thr (bisection over
//          the 65536 keys); m = number of r in [0, H) with M(tau) + r * E(tau) < thr
//          (H tokens of key tau, E(tau) their e value); kept: key > tau, or key ==
//          tau and fewer than m tokens of key tau precede it.  Without top-p every
//          token is kept.  w_j = e_j when kept, else 0; K = chunked total of w;
//          p'_j = w_j / K.
//   draw from a weight row r with x removed (x = -1: none): R = chunked total (if
//          R <= 0 the exclusion is dropped); t = u_draw * R; c* = first chunk with
//          prefix_c + R_c > t (prefix summed sequentially); j = first index in c*
//          with prefix_c* + q_j > t, q_j the sequential in-chunk sum from the chunk
//          start.  If no chunk qualifies (rounding), the last index with r_j > 0.
//   uniforms (both contracts): Philox4x32-10 (Salmon et al., SC'11), key = seed,
//          counter = (step lo, step hi, j / 4, 0), word j % 4, u = (word >> 8) * 2^-24;
//          j = i for guess i, j = 63 for the draw.
//   with draft rows (a draft model's distribution per guess): bf16 draft logits
//          give q' by the same procedure (same T and top-p); fp32 rows are
//          probabilities q used as given.  a = min(p'_g / max(q_g, 1e-12), 1);
//          a rejection draws from r_j = max(p'_j - q_j, 0) (p'_j = w_j / K one fp32
//          division, q'_j likewise, the difference one op), falling back to w when
//          r has no mass (verifier.py:44-56).
// FP contraction is disabled in this file's arithmetic so that every operation on
// these paths is a single IEEE-rounded fp32 op (exp3's fused multiply-adds are written
// out), as in the C oracle.
#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kThreads = 256;
constexpr int kChunks = 256;
constexpr int kMaxRows = 17;  // up to 16 guesses per sequence

#pragma clang fp contract(off)

__device__ float cephes_exp(float x) {
#pragma clang fp contract(off)
  if (x < -86.0f) return 0.0f;
  const float fx = floorf(1.44269504088896341f * x + 0.5f);
  float r = x - fx * 0.693359375f;
  r = r - fx * -2.12194440e-4f;
  const float z = r * r;
  float y = 1.9875691500E-4f * r + 1.3981999507E-3f;
  y = y * r + 8.3334519073E-3f;
  y = y * r + 4.1665795894E-2f;
  y = y * r + 1.6666665459E-1f;
  y = y * r + 5.0000001201E-1f;
  y = y * z + r + 1.0f;
  const int n = (int)fx;
  return y * __builtin_bit_cast(float, (uint32_t)(n + 127) << 23);
}

__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
  for (int round = 0; round < 10; ++round) {
    if (round > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k0;
    const uint32_t n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

__device__ float philox_uniform(uint64_t seed, uint64_t step, int j) {
  uint32_t c[4] = {(uint32_t)step, (uint32_t)(step >> 32), (uint32_t)(j >> 2), 0u};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  return (float)(c[j & 3] >> 8) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ uint64_t key_of(float v, uint32_t idx) {
  v = v + 0.0f;  // -0 compares equal to +0 (torch.argmax): give both one key
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

// 16-bit order key of a bf16 logit (larger logit, larger key; -0 as +0) and back
__device__ __forceinline__ uint32_t key16(uint16_t b) {
  if ((b & 0x7FFFu) == 0) b = 0;
  return (b & 0x8000u) ? (uint32_t)(~b & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}

__device__ __forceinline__ uint16_t bf16_of_key16(uint32_t k) {
  return (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)(~k & 0xFFFFu);
}

__device__ uint64_t block_max_u64(uint64_t v, uint64_t* s_red) {
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = v > w ? v : w;
  }
  __syncthreads();
  if (threadIdx.x % kWave == 0) s_red[threadIdx.x / kWave] = v;
  __syncthreads();
  uint64_t r = s_red[0];
  for (int w = 1; w < kThreads / kWave; ++w) r = r > s_red[w] ? r : s_red[w];
  return r;
}

__device__ float block_max_f32(float v, float* s_red) {
  v = wave_max(v);
  __syncthreads();
  if (threadIdx.x % kWave == 0) s_red[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = s_red[0];
  for (int w = 1; w < kThreads / kWave; ++w) r = fmaxf(r, s_red[w]);
  return r;
}

struct AcceptParams {
  const uint16_t* logits;
  int64_t ld;
  const uint64_t* partials;
  int num_tiles;
  int vocab;
  const int32_t* drafts;
  int max_drafts;
  const int32_t* num_drafts;
  const int32_t* row_start;
  const float* temperature;  // per sequence; null: every sequence greedy
  const float* top_p;        // per sequence; null: 1
  const uint64_t* seeds;
  const uint64_t* steps;
  int32_t* out_tokens;
  int32_t* num_out;
  int32_t* history;
  int64_t hist_stride;
  int32_t* history_len;
  int32_t* num_cached;
  const void* draft_rows;  // sampled: the draft's distribution per guess, or null (one-hot)
  int draft_dtype;         // NE_DTYPE_BF16: logits, NE_DTYPE_FP32: probabilities
  int64_t dld;
  const int32_t* draft_row_start;
  int rows_done;  // sampled one-hot rows decided by accept_rows_kernel (out_tokens holds them)
};

// greedy target of one row: argmax over bf16 logits or the LM-head partials
__device__ int row_argmax(const AcceptParams& p, int row, uint64_t* s_red) {
  uint64_t best = 0;
  if (p.logits != nullptr) {
    const uint16_t* src = p.logits + (int64_t)row * p.ld;
    for (int j = threadIdx.x; j < p.vocab; j += kThreads) {
      const uint64_t k = key_of(bf16_to_f32(src[j]), j);
      best = best > k ? best : k;
    }
  } else {
    const uint64_t* src = p.partials + (int64_t)row * p.num_tiles;
    for (int t = threadIdx.x; t < p.num_tiles; t += kThreads) best = best > src[t] ? best : src[t];
  }
  best = block_max_u64(best, s_red);
  return (int)(0xFFFFFFFFu - (uint32_t)best);
}

// ---- one row's distribution under the contract ------------------------------------
// LDS of a distribution: its kept-weight chunk sums and, with top-p, the number of
// threshold-key tokens before each chunk (the tie rank at the chunk's start).
struct DistLds {
  float chunk[kChunks];
  int tie_base[kChunks];
};

struct Dist {
  const uint16_t* row;
  float T, mx, total;
  bool topp;
  uint32_t tau;
  int m;
};

__device__ __forceinline__ int chunk_len(int V) { return (V + kChunks - 1) / kChunks; }

__device__ __forceinline__ float dist_e(const Dist& d, int j) {
  return cephes_exp(bf16_to_f32(d.row[j]) / d.T - d.mx);
}

// every thread: the sequential fp32 sum of v[0..255] (from LDS)
__device__ __forceinline__ float lds_total(const float* v) {
  float t = 0.f;
  for (int c = 0; c < kChunks; ++c) t = t + v[c];
  return t;
}

// M(v): chunked total of e over tokens with key > v (all threads; uniform result)
__device__ float masked_total(const Dist& d, int V, uint32_t v, float* s_tmp) {
  const int CH = chunk_len(V);
  const int lo = threadIdx.x * CH, hi = min(lo + CH, V);
  float s = 0.f;
  for (int j = lo; j < hi; ++j)
    if (key16(d.row[j]) > v) s = s + dist_e(d, j);
  __syncthreads();
  s_tmp[threadIdx.x] = s;
  __syncthreads();
  return lds_total(s_tmp);
}

// sets up d for `row`; leaves the kept chunk sums and tie bases in L
__device__ void dist_setup(Dist& d, const uint16_t* row, int V, float T, float top_p, DistLds& L, float* s_tmp,
                           float* s_redf) {
  d.row = row;
  d.T = T;
  float m = -INFINITY;
  for (int j = threadIdx.x; j < V; j += kThreads) m = fmaxf(m, bf16_to_f32(row[j]) / T);
  d.mx = block_max_f32(m, s_redf);
  d.topp = top_p < 1.0f;
  d.tau = 0;
  d.m = 0;
  const int CH = chunk_len(V);
  const int lo = threadIdx.x * CH, hi = min(lo + CH, V);
  float s = 0.f;
  for (int j = lo; j < hi; ++j) s = s + dist_e(d, j);
  __syncthreads();
  L.chunk[threadIdx.x] = s;
  __syncthreads();
  const float z = lds_total(L.chunk);
  d.total = z;
  if (!d.topp) return;
  const float thr = top_p * z;
  uint32_t a = 0, b = 65535;
  while (a < b) {  // uniform across the work-group
    const uint32_t mid = (a + b) / 2;
    if (masked_total(d, V, mid, s_tmp) < thr) b = mid; else a = mid + 1;
  }
  d.tau = a;
  const float mt = masked_total(d, V, a, s_tmp);
  int cnt = 0;
  for (int j = lo; j < hi; ++j) cnt += key16(row[j]) == a;
  __syncthreads();
  L.tie_base[threadIdx.x] = cnt;
  __syncthreads();
  int h = 0, base = 0;
  for (int c = 0; c < kChunks; ++c) {
    if (c == (int)threadIdx.x) base = h;
    h += L.tie_base[c];
  }
  const float e_tau = cephes_exp(bf16_to_f32(bf16_of_key16(a)) / T - d.mx);
  int r0 = 0, r1 = h;  // m = number of r in [0, h) with mt + r * e_tau < thr
  while (r0 < r1) {
    const int mid = (r0 + r1) / 2;
    if (mt + (float)mid * e_tau < thr) r0 = mid + 1; else r1 = mid;
  }
  d.m = r0;
  __syncthreads();
  L.tie_base[threadIdx.x] = base;
  // kept chunk sums
  float k = 0.f;
  int tie = base;
  for (int j = lo; j < hi; ++j) {
    const uint32_t key = key16(row[j]);
    const bool kept = key > d.tau || (key == d.tau && tie < d.m);
    tie += key == d.tau;
    if (kept) k = k + dist_e(d, j);
  }
  L.chunk[threadIdx.x] = k;
  __syncthreads();
  d.total = lds_total(L.chunk);
}

// scans one chunk in index order, calling f(j, w_j) with each token's kept weight until
// f returns false
template <typename F>
__device__ __forceinline__ void scan_chunk(const Dist& d, const DistLds& L, int V, int c, F&& f) {
  const int CH = chunk_len(V);
  const int lo = c * CH, hi = min(lo + CH, V);
  int tie = d.topp ? L.tie_base[c] : 0;
  for (int j = lo; j < hi; ++j) {
    bool kept = true;
    if (d.topp) {
      const uint32_t key = key16(d.row[j]);
      kept = key > d.tau || (key == d.tau && tie < d.m);
      tie += key == d.tau;
    }
    if (!f(j, kept ? dist_e(d, j) : 0.f)) return;
  }
}

// kept weight of token x (one thread)
__device__ float weight_at(const Dist& d, const DistLds& L, int V, int x) {
  float w = 0.f;
  scan_chunk(d, L, V, x / chunk_len(V), [&](int j, float wj) {
    if (j == x) {
      w = wj;
      return false;
    }
    return true;
  });
  return w;
}

// inverse-CDF draw from d's kept weights with token x removed (x < 0: none); one thread
__device__ int draw_dist(const Dist& d, const DistLds& L, int V, int x, float u) {
  const int CH = chunk_len(V);
  auto chunk_sum = [&](int c, int excl) -> float {
    if (excl < 0 || excl / CH != c) return L.chunk[c];
    float s = 0.f;
    scan_chunk(d, L, V, c, [&](int j, float wj) {
      s = s + (j == excl ? 0.f : wj);
      return true;
    });
    return s;
  };
  int excl = x;
  float R = 0.f;
  for (int c = 0; c < kChunks; ++c) R = R + chunk_sum(c, excl);
  if (!(R > 0.f)) {
    excl = -1;
    R = 0.f;
    for (int c = 0; c < kChunks; ++c) R = R + chunk_sum(c, excl);
  }
  const float t = u * R;
  float prefix = 0.f;
  for (int c = 0; c < kChunks; ++c) {
    const float rc = chunk_sum(c, excl);
    if (prefix + rc > t) {
      float q = 0.f;
      int res = -1;
      scan_chunk(d, L, V, c, [&](int j, float wj) {
        q = q + (j == excl ? 0.f : wj);
        if (prefix + q > t) {
          res = j;
          return false;
        }
        return true;
      });
      if (res >= 0) return res;
    }
    prefix = prefix + rc;
  }
  for (int c = kChunks - 1; c >= 0; --c) {
    int found = -1;
    scan_chunk(d, L, V, c, [&](int j, float wj) {
      if (j != excl && wj > 0.f) found = j;
      return true;
    });
    if (found >= 0) return found;
  }
  return 0;
}

// residual draw: r_j = max(p'_j - q_j, 0) over the target d and the draft (bf16 logits dq,
// or fp32 probabilities qp); every thread sums its chunk, thread 0 scans.  Falls back to
// the target's kept weights (no exclusion) when the residual has no mass.
__device__ int draw_residual(const Dist& d, const DistLds& L, const Dist& dq, const DistLds& Lq,
                             const float* qp, int V, float u, float* s_rchunk) {
  const int CH = chunk_len(V);
  // r over one chunk, in index order
  auto scan_r = [&](int c, auto&& f) {
    const int lo = c * CH, hi = min(lo + CH, V);
    int tie = d.topp ? L.tie_base[c] : 0;
    int tieq = (qp == nullptr && dq.topp) ? Lq.tie_base[c] : 0;
    for (int j = lo; j < hi; ++j) {
      bool kept = true;
      if (d.topp) {
        const uint32_t key = key16(d.row[j]);
        kept = key > d.tau || (key == d.tau && tie < d.m);
        tie += key == d.tau;
      }
      const float pj = kept ? dist_e(d, j) / d.total : 0.f;
      float qj;
      if (qp != nullptr) {
        qj = qp[j];
      } else {
        bool keptq = true;
        if (dq.topp) {
          const uint32_t key = key16(dq.row[j]);
          keptq = key > dq.tau || (key == dq.tau && tieq < dq.m);
          tieq += key == dq.tau;
        }
        qj = keptq ? dist_e(dq, j) / dq.total : 0.f;
      }
      const float r = pj - qj;
      if (!f(j, r > 0.f ? r : 0.f)) return;
    }
  };
  float sr = 0.f;
  scan_r((int)threadIdx.x, [&](int, float r) {
    sr = sr + r;
    return true;
  });
  __syncthreads();
  s_rchunk[threadIdx.x] = sr;
  __syncthreads();
  int res = 0;
  if (threadIdx.x == 0) {
    float R = 0.f;
    for (int c = 0; c < kChunks; ++c) R = R + s_rchunk[c];
    if (!(R > 0.f)) {
      res = draw_dist(d, L, V, -1, u);
    } else {
      const float t = u * R;
      float prefix = 0.f;
      res = -1;
      for (int c = 0; c < kChunks && res < 0; ++c) {
        const float rc = s_rchunk[c];
        if (prefix + rc > t) {
          float q = 0.f;
          scan_r(c, [&](int j, float r) {
            q = q + r;
            if (prefix + q > t) {
              res = j;
              return false;
            }
            return true;
          });
        }
        prefix = prefix + rc;
      }
      if (res < 0) {
        for (int c = kChunks - 1; c >= 0 && res < 0; --c)
          scan_r(c, [&](int j, float r) {
            if (r > 0.f) res = j;
            return true;
          });
        if (res < 0) res = 0;
      }
    }
  }
  return res;
}

// ---- integer-mass contract for one-hot guesses: one work-group per verify row -------
// Every token's weight depends only on its bf16 key: E(k) = floor(exp3(val(k) / T - max)
// * 2^31) (header).  The row's keys are counted once into an LDS histogram; the sum Z,
// the top-p threshold, the guess's acceptance and the draw's key all come from the
// histogram (exp3 once per occupied key), and integer sums make every parallel order
// give the oracle's result.  A draw then finds the r-th occurrence of its key in index
// order with one compare-only pass.  Row i of sequence b writes out_tokens[b][i]: -2
// when it keeps its guess, else the token it draws (the bonus row always draws); the
// finish in accept_kernel keeps the rows up to the first that drew.
constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / kWave;
constexpr int kKeysPerThread = 65536 / kRowThreads;
constexpr int kMaxWraps = 16;  // 16-bit count wraps recorded per row: vocab < 16 * 65536

struct RowLds {
  // counts of keys 2w (bits 0..15) and 2w + 1 (bits 16..31), modulo the wraps below
  uint32_t hist[32768];
  uint64_t seg_mass[kRowThreads];  // mass of keys [64 s, 64 s + 64)
  uint64_t wave_part[kRowWaves];
  uint32_t wrap_key[kMaxWraps];  // bit 31: the high half's running value (count of key +
  int n_wrap;                    //   low carries) crossed 65536; else the low half did
  uint32_t wrap_key_spare[kRowWaves];  // occupied segments per wave
  uint32_t wave_cnt[kRowWaves];        // tokens counted per wave's segments
  uint16_t seg_list[kRowThreads];      // occupied segments in order
  int n_seg;
  uint64_t k_total, above, want;
  uint32_t kmax, tau, m, kappa;
  int seg;
};

__device__ __forceinline__ float exp3(float x) {
  if (x < -86.0f) return 0.0f;
  const float fx = floorf(__builtin_fmaf(x, 1.44269504088896341f, 0.5f));
  float r = __builtin_fmaf(fx, -0.693359375f, x);
  r = __builtin_fmaf(fx, 2.12194440e-4f, r);
  float y = __builtin_fmaf(1.9875691500E-4f, r, 1.3981999507E-3f);
  y = __builtin_fmaf(y, r, 8.3334519073E-3f);
  y = __builtin_fmaf(y, r, 4.1665795894E-2f);
  y = __builtin_fmaf(y, r, 1.6666665459E-1f);
  y = __builtin_fmaf(y, r, 5.0000001201E-1f);
  const float z = r * r;
  y = __builtin_fmaf(y, z, r);
  y = y + 1.0f;
  const int n = (int)fx;
  return y * __builtin_bit_cast(float, (uint32_t)(n + 127) << 23);
}

// count of key k: its 16-bit half plus 65536 per recorded wrap (a high half's running
// value also holds the low half's carries, which the low half's own wraps count)
__device__ __forceinline__ uint32_t row_count(const RowLds& L, uint32_t k) {
  const uint32_t w = L.hist[k >> 1];
  uint32_t c = (k & 1) ? (w >> 16) : (w & 0xFFFFu);
  const int n = min(L.n_wrap, kMaxWraps);
  for (int i = 0; i < n; ++i) {
    const uint32_t e = L.wrap_key[i], ek = e & 0xFFFFu;
    if (e >> 31) {  // a high-half crossing of key ek (odd)
      if (ek == k) c += 65536u;
    } else if (ek == k) {  // a low-half wrap of key ek (even)
      c += 65536u;
    } else if ((k & 1) && ek == k - 1) {  // its carry went into key k's half
      c -= 1u;
    }
  }
  return c;
}

__device__ __forceinline__ uint32_t row_weight(uint32_t k, float invT, float mx) {
  const float e = exp3(bf16_to_f32(bf16_of_key16(k)) * invT - mx);
  return (uint32_t)(e * 2147483648.0f);
}

__device__ __forceinline__ uint64_t shfl_xor_u64v(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((uint32_t)v, o), hi = __shfl_xor((uint32_t)(v >> 32), o);
  return ((uint64_t)hi << 32) | lo;
}

// over the lanes of a wave: the sum of v over higher lanes (integers: any order)
__device__ __forceinline__ uint64_t wave_suffix_excl_u64(uint64_t v) {
  const int lane = threadIdx.x % kWave;
  uint64_t incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t lo = __shfl_down((uint32_t)incl, o), hi = __shfl_down((uint32_t)(incl >> 32), o);
    if (lane + o < kWave) incl += ((uint64_t)hi << 32) | lo;
  }
  return incl - v;
}

// exclusive sum over the work-group's threads (ascending) of a u64, and the total
__device__ __forceinline__ uint64_t row_scan_u64(uint64_t v, RowLds& L, uint64_t* total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  uint64_t incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t lo = __shfl_up((uint32_t)incl, o), hi = __shfl_up((uint32_t)(incl >> 32), o);
    if (lane >= o) incl += ((uint64_t)hi << 32) | lo;
  }
  __syncthreads();
  if (lane == kWave - 1) L.wave_part[wave] = incl;
  __syncthreads();
  uint64_t before = 0, all = 0;
  for (int w = 0; w < kRowWaves; ++w) {
    const uint64_t x = L.wave_part[w];
    before += w < wave ? x : 0;
    all += x;
  }
  *total = all;
  return before + incl - v;
}

__global__ __launch_bounds__(kRowThreads) void accept_rows_kernel(AcceptParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  RowLds& L = *(RowLds*)smem;
  const int R = p.max_drafts + 1;
  const int b = blockIdx.x / R;
  const int i = blockIdx.x % R;
  const int tid = threadIdx.x;
  const int lane = tid % kWave, wave = tid / kWave;
  const float T = p.temperature[b];
  if (!(T > 0.f)) return;                                        // greedy: accept_kernel
  if (p.history != nullptr && p.history_len[b] == 0) return;     // inactive slot
  const int g = min(max(p.num_drafts[b], 0), p.max_drafts);
  if (i > g) return;
  const int V = p.vocab;
  const uint16_t* row = p.logits + (int64_t)(p.row_start[b] + i) * p.ld;
  const float top_p = p.top_p != nullptr ? p.top_p[b] : 1.f;
  const bool topp = top_p < 1.0f;
  const int guess = i < g ? p.drafts[(int64_t)b * p.max_drafts + i] : -1;

  // ---- histogram of the row's keys.  First with adds that return nothing: a 16-bit half
  // that overflows goes unnoticed there, but then the halves no longer sum to V (a wrap
  // takes 65535 or 65536 off the sum), which the segment pass checks; only such a row is
  // counted again with adds that return the old word and record every wrap.
  auto add_key = [&](uint32_t k) { atomicAdd(&L.hist[k >> 1], 1u << ((k & 1) * 16)); };
  auto count_key = [&](uint32_t k) {
    const uint32_t sh = (k & 1) * 16;
    const uint32_t old = atomicAdd(&L.hist[k >> 1], 1u << sh);
    // a low half that was 0xFFFF wrapped (and carried into the high half); a high half's
    // running value crosses 65536 when it was 0xFFFF and gains 1 by this add or its carry
    const bool low_wrap = sh == 0 && (old & 0xFFFFu) == 0xFFFFu;
    const bool high_cross = (old >> 16) == 0xFFFFu && (sh == 16 || low_wrap);
    if (low_wrap || high_cross) {
      const int slot = atomicAdd(&L.n_wrap, (int)low_wrap + (int)high_cross);
      if (low_wrap && slot < kMaxWraps) L.wrap_key[slot] = k;
      if (high_cross && slot + (int)low_wrap < kMaxWraps) L.wrap_key[slot + (int)low_wrap] = (k | 1u) | 0x80000000u;
    }
  };
  auto histogram = [&](bool tracked) {
    auto add = [&](uint32_t k) {
      if (tracked)
        count_key(k);
      else
        add_key(k);
    };
    if ((((uintptr_t)row) & 15) == 0) {
      // 16-byte loads in batches of kHistLoads per thread, the next batch requested before
      // the current one is counted
      constexpr int kHistLoads = 4;
      const int nvec = V / 8;
      const uint4* rv = (const uint4*)row;
      uint4 qa[kHistLoads], qb[kHistLoads];
      auto load = [&](uint4 (&q)[kHistLoads], int v0) {
#pragma unroll
        for (int u = 0; u < kHistLoads; ++u) {
          const int v = v0 + u * kRowThreads;
          q[u] = v < nvec ? rv[v] : uint4{0u, 0u, 0u, 0u};
        }
      };
      auto count = [&](const uint4 (&q)[kHistLoads], int v0) {
#pragma unroll
        for (int u = 0; u < kHistLoads; ++u) {
          if (v0 + u * kRowThreads >= nvec) break;
          const uint32_t w4[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            add(key16((uint16_t)(w4[h] & 0xFFFFu)));
            add(key16((uint16_t)(w4[h] >> 16)));
          }
        }
      };
      constexpr int kBatch = kHistLoads * kRowThreads;
      load(qa, tid);
      for (int v0 = tid; v0 < nvec; v0 += 2 * kBatch) {
        load(qb, v0 + kBatch);
        count(qa, v0);
        load(qa, v0 + 2 * kBatch);
        count(qb, v0 + kBatch);
      }
      for (int j = nvec * 8 + tid; j < V; j += kRowThreads) add(key16(row[j]));
    } else {
      for (int j = tid; j < V; j += kRowThreads) add(key16(row[j]));
    }
  };

  // ---- segment tid (keys 64 tid .. 64 tid + 63): its 32 histogram words at once, its
  // largest key, whether any key is occupied, and the sum of its counts (a count that
  // wrapped to 0 in its 16-bit half is found through row_count once wraps are recorded)
  const uint32_t k0 = (uint32_t)tid * kKeysPerThread;
  bool occupied = false;
  uint32_t top = 0;  // largest occupied key + 1
  auto segment_pass = [&](bool tracked) {
    const uint4* hw = (const uint4*)(L.hist + tid * (kKeysPerThread / 2));
    uint32_t w[kKeysPerThread / 2];
#pragma unroll
    for (int q = 0; q < kKeysPerThread / 8; ++q) {
      const uint4 v = hw[q];
      w[4 * q] = v.x;
      w[4 * q + 1] = v.y;
      w[4 * q + 2] = v.z;
      w[4 * q + 3] = v.w;
    }
    top = 0;
    uint32_t sum = 0;
    if (!tracked || L.n_wrap == 0) {
#pragma unroll
      for (int j = 0; j < kKeysPerThread / 2; ++j) {
        if (w[j] & 0xFFFFu) top = k0 + 2 * j + 1;
        if (w[j] >> 16) top = k0 + 2 * j + 2;
        sum += (w[j] & 0xFFFFu) + (w[j] >> 16);
      }
    } else {
      for (int j = 0; j < kKeysPerThread; ++j)
        if (row_count(L, k0 + j)) top = k0 + j + 1;
    }
    occupied = top != 0;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    if (lane == 0) L.wave_cnt[wave] = sum;
  };
  for (bool tracked = false;; tracked = true) {
    for (int w = tid; w < 32768 / 4; w += kRowThreads) ((uint4*)L.hist)[w] = uint4{0u, 0u, 0u, 0u};
    if (tid == 0) L.n_wrap = 0;
    __syncthreads();
    histogram(tracked);
    __syncthreads();
    segment_pass(tracked);
    __syncthreads();
    uint32_t counted = 0;
    for (int w = 0; w < kRowWaves; ++w) counted += L.wave_cnt[w];
    if (tracked || counted == (uint32_t)V) break;
    __syncthreads();  // a 16-bit count overflowed: count again, recording wraps
  }
  {
    uint32_t m = top;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = max(m, (uint32_t)__shfl_xor(m, o));
    if (lane == 0) L.wave_part[wave] = m;
  }
  // occupied segments listed in order (their masses need exp3; the rest weigh 0)
  const uint64_t occ_mask = __builtin_amdgcn_ballot_w64(occupied);
  if (lane == 0) L.wrap_key_spare[wave] = (uint32_t)__builtin_popcountll(occ_mask);
  __syncthreads();
  if (tid == 0) {
    uint32_t mm = 0;
    for (int w = 0; w < kRowWaves; ++w) mm = max(mm, (uint32_t)L.wave_part[w]);
    L.kmax = mm - 1;
  }
  {
    uint32_t at = 0, n_occ = 0;
    for (int w = 0; w < kRowWaves; ++w) {
      at += w < wave ? L.wrap_key_spare[w] : 0u;
      n_occ += L.wrap_key_spare[w];
    }
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(occ_mask >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)occ_mask, 0u));
    if (occupied) L.seg_list[at + rank] = (uint16_t)tid;
    L.seg_mass[tid] = 0;
    if (tid == 0) L.n_seg = (int)n_occ;
  }
  __syncthreads();
  const uint32_t kmax = L.kmax;
  const float invT = 1.0f / T;
  const float mx = bf16_to_f32(bf16_of_key16(kmax)) * invT;
  // mass of key 64 s + lane (every lane of a wave, for one segment s)
  auto lane_mass = [&](int seg) -> uint64_t {
    const uint32_t k = (uint32_t)seg * kKeysPerThread + lane;
    const uint32_t c = row_count(L, k);
    return c ? (uint64_t)c * row_weight(k, invT, mx) : 0;
  };

  // ---- masses of the occupied segments: wave w takes list entries w, w + 16, ...
  for (int e = wave; e < L.n_seg; e += kRowWaves) {
    const int seg = L.seg_list[e];
    uint64_t mass = lane_mass(seg);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mass += shfl_xor_u64v(mass, o);
    if (lane == 0) L.seg_mass[seg] = mass;
  }
  __syncthreads();
  const uint64_t mine = L.seg_mass[tid];
  uint64_t z;
  const uint64_t below = row_scan_u64(mine, L, &z);
  const uint64_t above = z - below - mine;  // mass of the keys above segment tid

  // ---- top-p: thr, then tau in the segment where the mass above crosses it
  uint64_t thr = 0;
  if (topp) {
    thr = (uint64_t)((double)z * (double)top_p);
    thr = thr < 1 ? 1 : thr;
    if (above < thr && above + mine >= thr) {
      L.seg = tid;
      L.above = above;
    }
  }
  __syncthreads();
  if (tid < kWave) {
    if (topp) {
      const int seg = L.seg;
      const uint64_t mass = lane_mass(seg);
      const uint64_t run = L.above + wave_suffix_excl_u64(mass);  // M(key): mass above it
      const bool here = run < thr && run + mass >= thr;
      if (here) {
        const uint32_t k = (uint32_t)seg * kKeysPerThread + lane;
        const uint32_t c = row_count(L, k);
        const uint64_t e = row_weight(k, invT, mx);
        uint64_t m = (thr - run + e - 1) / e;
        m = m > c ? c : m;
        L.tau = k;
        L.m = (uint32_t)m;
        L.k_total = run + m * e;
      }
    } else if (tid == 0) {
      L.tau = 0;
      L.m = 0;
      L.k_total = z;
    }
  }
  __syncthreads();
  const uint32_t tau = L.tau, m_tau = L.m;
  const uint64_t K = L.k_total;

  // ---- the guess: its weight if kept (ties at tau kept when fewer than m precede it)
  uint64_t wg = 0;
  uint32_t kg = 0;
  if (guess >= 0) {
    // a guess outside the vocabulary weighs 0 (never kept, nothing removed from the draw)
    const bool valid = guess < V;
    kg = valid ? key16(row[guess]) : 0u;
    bool kept = valid && (!topp || kg > tau);
    if (valid && topp && kg == tau) {
      if (m_tau >= row_count(L, tau)) {
        kept = true;
      } else {  // its rank among key-tau tokens, counted over [0, guess)
        int mine_c = 0;
        for (int j = tid; j < guess; j += kRowThreads) mine_c += key16(row[j]) == tau;
        uint64_t rank;
        row_scan_u64((uint64_t)mine_c, L, &rank);
        kept = rank < m_tau;
      }
    }
    wg = kept ? row_weight(kg, invT, mx) : 0;
    const uint32_t u = (uint32_t)(philox_uniform(p.seeds[b], p.steps[b], i) * 16777216.0f);
    // kept iff w >= K or (w > 0 and u K < w 2^24): u K < 2^74, w 2^24 < 2^56
    const uint64_t lo = (uint64_t)u * K, hi = __umul64hi((uint64_t)u, K);
    if (wg >= K || (wg > 0 && hi == 0 && lo < (wg << 24))) {
      if (tid == 0) p.out_tokens[(int64_t)b * R + i] = -2;
      return;
    }
  }

  // ---- the draw: kept tokens by key (descending) then index, the guess removed
  int x = guess;
  uint64_t rw = K - wg;
  if (rw == 0) {  // the guess held all the kept weight: draw without removing it
    x = -1;
    wg = 0;
    rw = K;
  }
  const uint32_t ud = (uint32_t)(philox_uniform(p.seeds[b], p.steps[b], 63) * 16777216.0f);
  const uint64_t t = (uint64_t)ud * (rw >> 24) + (((uint64_t)ud * (rw & 0xFFFFFFu)) >> 24);
  const int seg_tau = topp ? (int)(tau / kKeysPerThread) : -1;
  const int seg_g = wg ? (int)(kg / kKeysPerThread) : -1;
  // kept mass of segment tid: all of it above tau's segment, K minus the mass above it
  // in tau's segment, none below; less the removed guess
  uint64_t kept_seg = mine;
  if (topp && tid < seg_tau) kept_seg = 0;
  if (tid == seg_tau) kept_seg = K - above;
  if (tid == seg_g) kept_seg -= wg;
  uint64_t tot;
  const uint64_t kb = row_scan_u64(kept_seg, L, &tot);
  const uint64_t ka = tot - kb - kept_seg;  // kept mass above segment tid
  if (ka <= t && t < ka + kept_seg) {
    L.seg = tid;
    L.above = ka;
  }
  __syncthreads();
  if (tid < kWave) {
    const int seg = L.seg;
    const uint32_t k = (uint32_t)seg * kKeysPerThread + lane;
    uint64_t c = (topp && k < tau) ? 0 : ((topp && k == tau) ? m_tau : row_count(L, k));
    if (wg && k == kg) c -= 1;
    const uint64_t e = c ? row_weight(k, invT, mx) : 0;
    const uint64_t w = c * e;
    const uint64_t run = L.above + wave_suffix_excl_u64(w);
    if (w && run <= t && t < run + w) {
      L.kappa = k;
      L.want = (t - run) / e;
    }
  }
  __syncthreads();
  // ---- the want-th occurrence of key kappa in index order, x skipped.  Wave w counts a
  // contiguous stretch of the row in chunks of kOccLoads loads per lane (8 tokens per lane
  // per 16-byte load, a chunk's loads requested together), keeping each load's hit bits;
  // the waves' counts are summed in order, and the wave holding the token finds it from
  // the bits (a stretch of more than one chunk loads the chunks again).
  const uint32_t kappa = L.kappa;
  const uint64_t want = L.want;
  // 16-byte loads need an aligned row whose length is a multiple of 8 (no load crosses V)
  const bool vec = (((uintptr_t)row) & 15) == 0 && (V & 7) == 0;
  const int step_t = vec ? 8 * kWave : kWave;  // tokens per wave per load
  const int span = ((V + kRowWaves - 1) / kRowWaves + step_t - 1) / step_t * step_t;
  const int w_lo = wave * span, w_hi = min(w_lo + span, V);
  // The bf16 bit patterns of key kappa (two for the key of -0 and +0), compared two tokens
  // per 32-bit word: half_zero marks each 16-bit half of v that is 0 with its top bit.
  const uint32_t pat = bf16_of_key16(kappa);  // +0 for the key of -0 and +0
  const bool zero_key = kappa == 0x8000u;
  const uint32_t p1 = pat * 0x10001u, p2 = 0x80008000u;
  auto half_zero = [](uint32_t v) -> uint32_t { return ~(((v & 0x7FFF7FFFu) + 0x7FFF7FFFu) | v) & 0x80008000u; };
  // hits among this lane's tokens j0 + 8 lane .. +8 (vec; bit h for token h) or j0 + lane
  auto lane_hits = [&](int j0, const uint4& q) -> uint32_t {
    if (vec) {
      const int j = j0 + 8 * lane;
      if (j >= w_hi) return 0u;
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
      uint32_t m = 0;  // token 2c in bit 2c, token 2c + 1 in bit 16 + 2c
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        uint32_t z = half_zero(w4[c] ^ p1);
        if (zero_key) z |= half_zero(w4[c] ^ p2);
        m |= z >> (15 - 2 * c);
      }
      uint32_t bits = (m | (m >> 15)) & 0xFFu;
      if ((uint32_t)(x - j) < 8u) bits &= ~(1u << (x - j));
      return bits;
    }
    const int j = j0 + lane;
    return (uint32_t)(j < w_hi && j != x && key16(row[j]) == kappa);
  };
  constexpr int kOccLoads = 20;
  constexpr int kOccHalf = kOccLoads / 2;
  const int chunk_t = kOccLoads * step_t;  // tokens per wave per chunk
  const int n_chunks = (w_hi - w_lo + chunk_t - 1) / chunk_t;
  uint32_t hb[kOccLoads / 4];  // load u's hit bits in byte u % 4 of hb[u / 4]
  // chunk c's hit bits into hb, two half-chunks of loads in flight; returns the lane's hits
  auto chunk_bits = [&](int c) -> uint32_t {
    uint32_t n = 0;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      uint4 q[kOccHalf];
#pragma unroll
      for (int u = 0; u < kOccHalf; ++u) {
        const int j0 = w_lo + c * chunk_t + (hh * kOccHalf + u) * step_t;
        const int j = j0 + (vec ? 8 * lane : lane);
        q[u] = (vec && j < w_hi) ? *(const uint4*)(row + j) : uint4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < kOccHalf; ++u) {
        const int uu = hh * kOccHalf + u;
        const int j0 = w_lo + c * chunk_t + uu * step_t;
        const uint32_t bits = j0 < w_hi ? lane_hits(j0, q[u]) : 0u;
        if (uu % 4 == 0) hb[uu / 4] = 0;
        hb[uu / 4] |= bits << (8 * (uu % 4));
        n += __builtin_popcount(bits);
      }
    }
    return n;
  };
  uint32_t occ = 0;
  for (int c = 0; c < n_chunks; ++c) occ += chunk_bits(c);
  uint32_t wocc = occ;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wocc += __shfl_xor(wocc, o);
  if (lane == 0) L.wave_part[wave] = wocc;
  __syncthreads();
  uint64_t before = 0;
  for (int w = 0; w < wave; ++w) before += L.wave_part[w];
  if (before <= want && want < before + wocc) {  // uniform within the wave
    uint64_t seen = before;
    for (int c = 0; c < n_chunks; ++c) {
      if (n_chunks > 1) chunk_bits(c);  // one chunk: its bits are still in hb
      bool found = false;
#pragma unroll
      for (int wi = 0; wi < kOccLoads / 4 && !found; ++wi)
#pragma unroll 1
      for (int uu = 4 * wi; uu < 4 * wi + 4; ++uu) {
        const uint32_t bits = (hb[wi] >> (8 * (uu % 4))) & 0xFFu;
        const uint32_t n = __builtin_popcount(bits);
        uint32_t incl = n;  // inclusive scan of the lanes' counts
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
          const uint32_t t2 = __shfl_up(incl, o);
          if (lane >= o) incl += t2;
        }
        const uint32_t total = __shfl(incl, kWave - 1);
        if (want < seen + total) {  // uniform
          const uint64_t start_l = seen + incl - n;
          if (start_l <= want && want < start_l + n) {
            uint32_t r = (uint32_t)(want - start_l), bb = bits;
            for (uint32_t q = 0; q < r; ++q) bb &= bb - 1;  // drop the r lowest hits
            const int h = __builtin_ctz(bb);
            const int j0 = w_lo + c * chunk_t + uu * step_t;
            p.out_tokens[(int64_t)b * R + i] = vec ? j0 + 8 * lane + h : j0 + lane;
          }
          found = true;
          break;
        }
        seen += total;
      }
      if (found) break;
    }
  }
}

__global__ __launch_bounds__(kThreads) void accept_kernel(AcceptParams p) {
  __shared__ uint64_t s_red[kThreads / kWave];
  __shared__ uint64_t s_rows[kMaxRows][kThreads / kWave];
  __shared__ float s_redf[kThreads / kWave];
  __shared__ DistLds s_d, s_dq;
  __shared__ float s_tmp[kChunks];
  __shared__ int s_target[kMaxRows];
  __shared__ int s_kept, s_final;
  __shared__ float s_accept;
  static_assert(kMaxRows <= kWave, "one lane of wave 0 per row");

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  // the sequence's scalars and thread i's guess (i < max_drafts) are requested together:
  // one memory round trip before the LM-head partials
  const int len = p.history != nullptr ? p.history_len[b] : 0;
  const int nd = p.num_drafts[b];
  const int rs0 = p.row_start[b];
  const float T = p.temperature != nullptr ? p.temperature[b] : 0.f;
  const int32_t* dr = p.drafts + (int64_t)b * p.max_drafts;
  const int my_draft = tid < p.max_drafts ? dr[tid] : 0;
  if (p.history != nullptr && len == 0) {  // inactive sequence slot
    if (tid <= p.max_drafts) p.out_tokens[(int64_t)b * (p.max_drafts + 1) + tid] = -1;
    if (tid == 0) p.num_out[b] = 0;
    return;
  }
  // a draft count beyond max_drafts would index past s_target and the draft row
  const int g = min(max(nd, 0), p.max_drafts);
  const int V = p.vocab;

  if (!(T > 0.f)) {
    if (p.logits == nullptr) {
      // the rows' LM-head partials are loaded together and reduced together: one
      // memory round trip and one barrier for all of them
      uint64_t best[kMaxRows];
      if (p.num_tiles <= 2 * kThreads) {  // the LM head's 512 keys per row: two per thread
        uint64_t v[kMaxRows][2];
#pragma unroll
        for (int i = 0; i < kMaxRows; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int t = tid + j * kThreads;
            v[i][j] = (i <= g && t < p.num_tiles) ? p.partials[(int64_t)(rs0 + i) * p.num_tiles + t] : 0;
          }
#pragma unroll
        for (int i = 0; i < kMaxRows; ++i) best[i] = v[i][0] > v[i][1] ? v[i][0] : v[i][1];
      } else {
#pragma unroll
        for (int i = 0; i < kMaxRows; ++i) {
          best[i] = 0;
          if (i <= g) {
            const uint64_t* src = p.partials + (int64_t)(rs0 + i) * p.num_tiles;
            for (int t = tid; t < p.num_tiles; t += kThreads) best[i] = best[i] > src[t] ? best[i] : src[t];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kMaxRows; ++i) {
        if (i <= g) {  // uniform
          uint64_t v = best[i];
#pragma unroll
          for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)v, o);
            const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o);
            const uint64_t w = ((uint64_t)hi << 32) | lo;
            v = v > w ? v : w;
          }
          if (tid % kWave == 0) s_rows[i][tid / kWave] = v;
        }
      }
      __syncthreads();
      if (tid <= g) {  // lane i of wave 0 finishes row i
        uint64_t r = s_rows[tid][0];
#pragma unroll
        for (int w = 1; w < kThreads / kWave; ++w) r = r > s_rows[tid][w] ? r : s_rows[tid][w];
        s_target[tid] = (int)(0xFFFFFFFFu - (uint32_t)r);
      }
    } else {
      for (int i = 0; i <= g; ++i) {
        const int t = row_argmax(p, rs0 + i, s_red);
        if (tid == 0) s_target[i] = t;
      }
    }
    __syncthreads();
    if (tid < kWave) {
      // kept = the number of leading guesses equal to their row's target (bit g of the
      // ballot is clear, so kept <= g)
      const uint64_t same = __builtin_amdgcn_ballot_w64(tid < g && my_draft == s_target[tid]);
      if (tid == 0) {
        const int kept = __builtin_ctzll(~same);
        s_kept = kept;
        s_final = s_target[kept];
      }
    }
    __syncthreads();
  } else if (p.rows_done) {
    // rows decided by accept_rows_kernel: -2 where the row kept its guess, else the token
    // it drew; the sequence keeps guesses up to the first row that drew
    if (tid <= g) s_target[tid] = p.out_tokens[(int64_t)b * (p.max_drafts + 1) + tid];
    __syncthreads();
    if (tid == 0) {
      int k = 0;
      while (k < g && s_target[k] == -2) ++k;
      s_kept = k;
      s_final = s_target[k];
    }
    __syncthreads();
  } else {
    const float top_p = p.top_p != nullptr ? p.top_p[b] : 1.f;
    const uint64_t seed = p.seeds[b], step = p.steps[b];
    const int dr0 = p.draft_rows != nullptr ? p.draft_row_start[b] : 0;
    const bool draft_logits = p.draft_rows != nullptr && p.draft_dtype == NE_DTYPE_BF16;
    int kept = 0;
    bool done = false;
    Dist d{}, dq{};
    for (int i = 0; i < g && !done; ++i) {
      dist_setup(d, p.logits + (int64_t)(rs0 + i) * p.ld, V, T, top_p, s_d, s_tmp, s_redf);
      const int guess = dr[i];
      const float u = philox_uniform(seed, step, i);
      const float* qp = nullptr;
      if (draft_logits)
        dist_setup(dq, (const uint16_t*)p.draft_rows + (int64_t)(dr0 + i) * p.dld, V, T, top_p, s_dq, s_tmp,
                   s_redf);
      else if (p.draft_rows != nullptr)
        qp = (const float*)p.draft_rows + (int64_t)(dr0 + i) * p.dld;
      // the acceptance test is made by thread 0 (the weight scans are serial) and broadcast
      if (tid == 0) {
        const float wg = weight_at(d, s_d, V, guess);
        const float pg = wg > 0.f ? wg / d.total : 0.f;
        float a = pg;
        if (draft_logits) {
          const float wq = weight_at(dq, s_dq, V, guess);
          const float q = wq > 0.f ? wq / dq.total : 0.f;
          a = fminf(pg / fmaxf(q, 1e-12f), 1.f);
        } else if (qp != nullptr) {
          a = fminf(pg / fmaxf(qp[guess], 1e-12f), 1.f);
        }
        s_accept = a;
      }
      __syncthreads();
      const float a = s_accept;
      if (a >= 1.f || (a > 0.f && u < a)) {
        ++kept;
        continue;
      }
      const float u_draw = philox_uniform(seed, step, 63);
      if (p.draft_rows == nullptr) {
        if (tid == 0) s_final = draw_dist(d, s_d, V, guess, u_draw);
      } else {
        const int t = draw_residual(d, s_d, dq, s_dq, qp, V, u_draw, s_tmp);
        if (tid == 0) s_final = t;
      }
      done = true;
    }
    if (!done) {
      dist_setup(d, p.logits + (int64_t)(rs0 + g) * p.ld, V, T, top_p, s_d, s_tmp, s_redf);
      if (tid == 0) s_final = draw_dist(d, s_d, V, -1, philox_uniform(seed, step, 63));
    }
    if (tid == 0) s_kept = kept;
    __syncthreads();
  }

  const int kept = s_kept;
  const int fin = s_final;
  // thread i writes token i (kept < g <= max_drafts, so my_draft holds guess i < kept)
  if (tid <= p.max_drafts)
    p.out_tokens[(int64_t)b * (p.max_drafts + 1) + tid] = (tid < kept) ? my_draft : (tid == kept ? fin : -1);
  if (tid == 0) p.num_out[b] = kept + 1;
  if (p.history != nullptr) {
    // a history row holds hist_stride tokens: tokens past it are not written (the host
    // refuses requests whose prompt + max_new_tokens exceed the rows' capacity)
    const int room = (int)min((int64_t)(kept + 1), max(p.hist_stride - len, (int64_t)0));
    int32_t* h = p.history + (int64_t)b * p.hist_stride;
    if (tid < room) h[len + tid] = (tid < kept) ? my_draft : fin;
    __syncthreads();
    if (tid == 0) {
      p.history_len[b] = len + room;
      if (p.num_cached != nullptr) p.num_cached[b] = len + kept;
    }
  }
}

}  // namespace

}  // namespace ne

using namespace ne;

extern "C" int ne_accept(const void* logits, int64_t ld_logits, const uint64_t* argmax_partials,
                         int32_t num_tiles, int32_t vocab, const int32_t* drafts, int32_t max_drafts,
                         const int32_t* num_drafts, const int32_t* row_start, int32_t num_seqs,
                         const float* temperature, const float* top_p, int32_t any_sampled,
                         const uint64_t* seeds, const uint64_t* steps, int32_t* out_tokens,
                         int32_t* num_out, int32_t* history, int64_t history_stride,
                         int32_t* history_len, int32_t* num_cached, const void* draft_rows,
                         int32_t draft_dtype, int64_t ld_draft, const int32_t* draft_row_start,
                         void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(vocab > 0, "vocab must be positive");
  NE_CHECK_ARG(drafts && num_drafts && row_start && out_tokens && num_out, "null pointer argument");
  NE_CHECK_ARG(max_drafts >= 1 && max_drafts < kMaxRows, "max_drafts must be in [1, %d]",
               kMaxRows - 1);
  NE_CHECK_ARG(logits || (argmax_partials && num_tiles > 0),
               "acceptance needs logits or argmax partials");
  if (any_sampled) {
    NE_CHECK_ARG(temperature != nullptr, "sampled acceptance needs per-sequence temperatures");
    NE_CHECK_ARG(logits != nullptr, "sampled acceptance needs logits");
    NE_CHECK_ARG(seeds && steps, "sampled acceptance needs seeds and steps");
  }
  NE_CHECK_ARG(!logits || ld_logits >= vocab, "ld_logits < vocab");
  NE_CHECK_ARG(!history || (history_len && history_stride > 0), "history needs history_len");
  NE_CHECK_ARG(!draft_rows || (any_sampled && draft_row_start && ld_draft >= vocab &&
                               (draft_dtype == NE_DTYPE_BF16 || draft_dtype == NE_DTYPE_FP32)),
               "draft rows need sampled sequences, draft_row_start, ld_draft >= vocab and a bf16 or "
               "fp32 dtype");
  AcceptParams p{};
  p.logits = (const uint16_t*)logits;
  p.ld = ld_logits;
  p.partials = argmax_partials;
  p.num_tiles = num_tiles;
  p.vocab = vocab;
  p.drafts = drafts;
  p.max_drafts = max_drafts;
  p.num_drafts = num_drafts;
  p.row_start = row_start;
  p.temperature = any_sampled ? temperature : nullptr;
  p.top_p = top_p;
  p.seeds = seeds;
  p.steps = steps;
  p.out_tokens = out_tokens;
  p.num_out = num_out;
  p.history = history;
  p.hist_stride = history_stride;
  p.history_len = history_len;
  p.num_cached = num_cached;
  p.draft_rows = draft_rows;
  p.draft_dtype = draft_dtype;
  p.dld = ld_draft;
  p.draft_row_start = draft_row_start;
  if (any_sampled && draft_rows == nullptr) {
    // one-hot guesses under the integer-mass contract: every sampled row decided by its
    // own work-group first, then the per-sequence finish
    NE_CHECK_SUPPORTED(vocab <= kMaxWraps / 2 * 65536, "sampled acceptance supports a vocabulary up to %d (got %d)",
                       kMaxWraps / 2 * 65536, vocab);
    static const hipError_t attr = hipFuncSetAttribute((const void*)accept_rows_kernel,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(RowLds));
    if (attr != hipSuccess) {
      set_error("accept: cannot reserve %d bytes of LDS: %s", (int)sizeof(RowLds), hipGetErrorString(attr));
      return NE_ELAUNCH;
    }
    p.rows_done = 1;
    hipLaunchKernelGGL(accept_rows_kernel, dim3((unsigned)num_seqs * (unsigned)(max_drafts + 1)), dim3(kRowThreads),
                       sizeof(RowLds), (hipStream_t)stream, p);
    const int rc = check_launch("accept_rows");
    if (rc != NE_OK) return rc;
  }
  hipLaunchKernelGGL(accept_kernel, dim3(num_seqs), dim3(kThreads), 0, (hipStream_t)stream, p);
  return check_launch("accept");
}
