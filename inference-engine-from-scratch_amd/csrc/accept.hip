// Fused acceptance for speculative verify on gfx950: greedy match or
// rejection sampling, correction/bonus token, KV-count rollback and history
// append, one 256-thread work-group per sequence.
//
// Restates verify_proposal (ne/engine/speculative/verifier.py:27-60) for the
// n-gram proposer, whose draft distribution is one-hot: the acceptance
// probability of guess g is min(1, p[g]), the residual max(p - onehot(g), 0)
// is p with g removed, and the rollback is num_cached = len_before + kept
// (ne/engine/speculative/speculative_generator.py:78-83).
//
// Greedy (temperature 0, ne/engine/sampling.py:32-34): target token of a row is
// the argmax of its bf16 logits, first index on ties (torch.argmax order).
//
// Sampled contract (temperature T > 0).  The reference draws with
// torch.rand / torch.multinomial, which no other implementation reproduces;
// this build fixes an explicit, order-defined procedure instead, shared bit for
// bit with the CPU oracle:
//   z_j  = fp32(logit_j) / T                  (IEEE fp32 division)
//   e_j  = cephes_exp(z_j - max_j z_j)        (Cephes expf, Moshier; 0 below -86)
//   S_c  = sequential fp32 sum of e_j over chunk c = [c*CH, min((c+1)*CH, V)),
//          CH = ceil(V / 256), c = 0..255;  Z = sequential sum of S_0..S_255
//   guess g of row i is kept iff p >= 1 or (p > 0 and u_i < p), p = e_g / Z
//   draw from row r excluding x (x = -1: none): r_j = e_j, r_x = 0; chunk sums
//          R_c and total R as above (if R <= 0 the exclusion is dropped);
//          t = u_draw * R; c* = first chunk with prefix_c + R_c > t (prefix
//          summed sequentially); j = first index in c* with prefix_c* + q_j > t,
//          q_j the sequential in-chunk sum from the chunk start.  If no chunk
//          qualifies (rounding), the last index with r_j > 0 is taken.
//   uniforms: Philox4x32-10 (Salmon et al., SC'11), key = seed, counter =
//          (step lo, step hi, j / 4, 0), word j % 4, u = (word >> 8) * 2^-24;
//          j = i for guess i, j = 63 for the draw.
//   with draft rows (a draft model's logits for each guess, the same T): f_j and
//          Zq as e_j and Z over the draft row; p = e_g / Z, q = max(f_g / Zq, 1e-12),
//          a = min(p / q, 1); guess i is kept iff a >= 1 or (a > 0 and u_i < a)
//          (verifier.py:44-51).  At the first rejection the draw is from the
//          residual r_j = max(e_j / Z - f_j / Zq, 0) (each term one fp32 op), chunk
//          sums and total as above, falling back to e when the total is not > 0
//          (verifier.py:52-56).
// FP contraction is disabled in this file's arithmetic on that path so that
// every operation is a single IEEE-rounded fp32 op, as in the C oracle.
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
  int mode;
  const uint16_t* logits;
  int64_t ld;
  const uint64_t* partials;
  int num_tiles;
  int vocab;
  const int32_t* drafts;
  int max_drafts;
  const int32_t* num_drafts;
  const int32_t* row_start;
  float temperature;
  const uint64_t* seeds;
  const uint64_t* steps;
  int32_t* out_tokens;
  int32_t* num_out;
  int32_t* history;
  int64_t hist_stride;
  int32_t* history_len;
  int32_t* num_cached;
  const uint16_t* draft_logits;  // sampled mode: the draft's row per guess, or null (one-hot)
  int64_t dld;
  const int32_t* draft_row_start;
};

__device__ __forceinline__ float logit_at(const AcceptParams& p, int row, int j) {
  return bf16_to_f32(p.logits[(int64_t)row * p.ld + j]);
}

// greedy target of one row: argmax over bf16 logits or the LM-head partials
__device__ int row_argmax(const AcceptParams& p, int row, uint64_t* s_red) {
  uint64_t best = 0;
  if (p.logits != nullptr) {
    for (int j = threadIdx.x; j < p.vocab; j += kThreads)
      best = best > key_of(logit_at(p, row, j), j) ? best : key_of(logit_at(p, row, j), j);
  } else {
    const uint64_t* src = p.partials + (int64_t)row * p.num_tiles;
    for (int t = threadIdx.x; t < p.num_tiles; t += kThreads) best = best > src[t] ? best : src[t];
  }
  best = block_max_u64(best, s_red);
  return (int)(0xFFFFFFFFu - (uint32_t)best);
}

// fp32 softmax pieces of one row under the fixed-order contract
struct RowSums {
  float mx;  // max z
  float Z;   // total of chunk sums
};

__device__ __forceinline__ float logit_of(const uint16_t* base, int64_t ld, int row, int j) {
  return bf16_to_f32(base[(int64_t)row * ld + j]);
}

// over the target's logits (base = p.logits) or the draft's (base = p.draft_logits)
__device__ RowSums row_sums(const AcceptParams& p, const uint16_t* base, int64_t ld, int row, float* s_chunk,
                            float* s_redf) {
  const int V = p.vocab;
  const int CH = (V + kChunks - 1) / kChunks;
  float m = -INFINITY;
  for (int j = threadIdx.x; j < V; j += kThreads) m = fmaxf(m, logit_of(base, ld, row, j) / p.temperature);
  const float mx = block_max_f32(m, s_redf);
  const int c = threadIdx.x;
  float s = 0.f;
  const int lo = c * CH, hi = min(lo + CH, V);
  for (int j = lo; j < hi; ++j) s = s + cephes_exp(logit_of(base, ld, row, j) / p.temperature - mx);
  s_chunk[c] = s;
  __syncthreads();
  float Z = 0.f;
  for (int k = 0; k < kChunks; ++k) Z = Z + s_chunk[k];
  __syncthreads();
  return RowSums{mx, Z};
}

// inverse-CDF draw excluding index x (x < 0: none); run after row_sums(row)
// left the chunk sums in s_chunk.  Executed by thread 0 only.
__device__ int draw_row(const AcceptParams& p, int row, const RowSums& rs, int x, float u,
                        const float* s_chunk) {
  const int V = p.vocab;
  const int CH = (V + kChunks - 1) / kChunks;
  const float T = p.temperature;
  auto r_at = [&](int j, int excl) -> float {
    return (j == excl) ? 0.f : cephes_exp(logit_at(p, row, j) / T - rs.mx);
  };
  auto chunk_sum = [&](int c, int excl) -> float {
    if (excl < 0 || excl / CH != c) return s_chunk[c];
    float s = 0.f;
    const int lo = c * CH, hi = min(lo + CH, V);
    for (int j = lo; j < hi; ++j) s = s + r_at(j, excl);
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
      const int lo = c * CH, hi = min(lo + CH, V);
      for (int j = lo; j < hi; ++j) {
        q = q + r_at(j, excl);
        if (prefix + q > t) return j;
      }
    }
    prefix = prefix + rc;
  }
  for (int j = V - 1; j >= 0; --j)
    if (r_at(j, excl) > 0.f) return j;
  return 0;
}

// residual draw: r_j = max(e_j / Z - f_j / Zq, 0) over the target row `row` (sums rs)
// and the draft row `drow` (sums rq); every thread sums its chunk, thread 0 scans.
// Falls back to the target row (no exclusion) when the residual total is not > 0.
__device__ int draw_residual(const AcceptParams& p, int row, const RowSums& rs, int drow, const RowSums& rq,
                             float u, float* s_chunk, float* s_rchunk) {
  const int V = p.vocab;
  const int CH = (V + kChunks - 1) / kChunks;
  const float T = p.temperature;
  auto r_at = [&](int j) -> float {
    const float pj = cephes_exp(logit_at(p, row, j) / T - rs.mx) / rs.Z;
    const float qj = cephes_exp(logit_of(p.draft_logits, p.dld, drow, j) / T - rq.mx) / rq.Z;
    const float r = pj - qj;
    return r > 0.f ? r : 0.f;
  };
  {
    const int c = threadIdx.x;
    float sr = 0.f;
    const int lo = c * CH, hi = min(lo + CH, V);
    for (int j = lo; j < hi; ++j) sr = sr + r_at(j);
    s_rchunk[c] = sr;
  }
  __syncthreads();
  int res = 0;
  if (threadIdx.x == 0) {
    float R = 0.f;
    for (int c = 0; c < kChunks; ++c) R = R + s_rchunk[c];
    if (!(R > 0.f)) {
      res = draw_row(p, row, rs, -1, u, s_chunk);
    } else {
      const float t = u * R;
      float prefix = 0.f;
      res = -1;
      for (int c = 0; c < kChunks && res < 0; ++c) {
        const float rc = s_rchunk[c];
        if (prefix + rc > t) {
          float q = 0.f;
          const int lo = c * CH, hi = min(lo + CH, V);
          for (int j = lo; j < hi; ++j) {
            q = q + r_at(j);
            if (prefix + q > t) {
              res = j;
              break;
            }
          }
        }
        prefix = prefix + rc;
      }
      if (res < 0) {
        for (int j = V - 1; j >= 0; --j)
          if (r_at(j) > 0.f) {
            res = j;
            break;
          }
        if (res < 0) res = 0;
      }
    }
  }
  return res;
}

__global__ __launch_bounds__(kThreads) void accept_kernel(AcceptParams p) {
  __shared__ uint64_t s_red[kThreads / kWave];
  __shared__ float s_redf[kThreads / kWave];
  __shared__ float s_chunk[kChunks];
  __shared__ float s_qchunk[kChunks];
  __shared__ int s_target[kMaxRows];
  __shared__ int s_kept, s_final;

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  if (p.history != nullptr && p.history_len[b] == 0) {  // inactive sequence slot
    for (int i = tid; i <= p.max_drafts; i += kThreads)
      p.out_tokens[(int64_t)b * (p.max_drafts + 1) + i] = -1;
    if (tid == 0) p.num_out[b] = 0;
    return;
  }
  // a draft count beyond max_drafts would index past s_target and the draft row
  const int g = min(max(p.num_drafts[b], 0), p.max_drafts);
  const int rs0 = p.row_start[b];
  const int32_t* dr = p.drafts + (int64_t)b * p.max_drafts;

  if (p.mode == NE_ACCEPT_GREEDY) {
    for (int i = 0; i <= g; ++i) {
      const int t = row_argmax(p, rs0 + i, s_red);
      if (tid == 0) s_target[i] = t;
    }
    __syncthreads();
    if (tid == 0) {
      int kept = 0;
      while (kept < g && dr[kept] == s_target[kept]) ++kept;
      s_kept = kept;
      s_final = s_target[kept];
    }
    __syncthreads();
  } else {
    const uint64_t seed = p.seeds[b], step = p.steps[b];
    int kept = 0;
    bool done = false;
    const int dr0 = p.draft_logits != nullptr ? p.draft_row_start[b] : 0;
    for (int i = 0; i < g && !done; ++i) {
      const RowSums rs = row_sums(p, p.logits, p.ld, rs0 + i, s_chunk, s_redf);
      const int guess = dr[i];
      const float pg = cephes_exp(logit_at(p, rs0 + i, guess) / p.temperature - rs.mx) / rs.Z;
      const float u = philox_uniform(seed, step, i);
      if (p.draft_logits == nullptr) {
        if (pg >= 1.f || (pg > 0.f && u < pg)) {
          ++kept;
          continue;
        }
        if (tid == 0) {
          s_final = draw_row(p, rs0 + i, rs, guess, philox_uniform(seed, step, 63), s_chunk);
        }
      } else {
        const RowSums rq = row_sums(p, p.draft_logits, p.dld, dr0 + i, s_qchunk, s_redf);
        const float qg = fmaxf(
            cephes_exp(logit_of(p.draft_logits, p.dld, dr0 + i, guess) / p.temperature - rq.mx) / rq.Z, 1e-12f);
        const float a = fminf(pg / qg, 1.f);
        if (a >= 1.f || (a > 0.f && u < a)) {
          ++kept;
          continue;
        }
        const int t = draw_residual(p, rs0 + i, rs, dr0 + i, rq, philox_uniform(seed, step, 63), s_chunk,
                                    s_qchunk);
        if (tid == 0) s_final = t;
      }
      done = true;
    }
    if (!done) {
      const RowSums rs = row_sums(p, p.logits, p.ld, rs0 + g, s_chunk, s_redf);
      if (tid == 0) s_final = draw_row(p, rs0 + g, rs, -1, philox_uniform(seed, step, 63), s_chunk);
    }
    if (tid == 0) s_kept = kept;
    __syncthreads();
  }

  const int kept = s_kept;
  const int fin = s_final;
  for (int i = tid; i <= p.max_drafts; i += kThreads)
    p.out_tokens[(int64_t)b * (p.max_drafts + 1) + i] = (i < kept) ? dr[i] : (i == kept ? fin : -1);
  if (tid == 0) p.num_out[b] = kept + 1;
  if (p.history != nullptr) {
    const int len = p.history_len[b];
    int32_t* h = p.history + (int64_t)b * p.hist_stride;
    for (int i = tid; i <= kept; i += kThreads) h[len + i] = (i < kept) ? dr[i] : fin;
    __syncthreads();
    if (tid == 0) {
      p.history_len[b] = len + kept + 1;
      if (p.num_cached != nullptr) p.num_cached[b] = len + kept;
    }
  }
}

}  // namespace

}  // namespace ne

using namespace ne;

extern "C" int ne_accept(int32_t mode, const void* logits, int64_t ld_logits,
                         const uint64_t* argmax_partials, int32_t num_tiles, int32_t vocab,
                         const int32_t* drafts, int32_t max_drafts, const int32_t* num_drafts,
                         const int32_t* row_start, int32_t num_seqs, float temperature,
                         const uint64_t* seeds, const uint64_t* steps, int32_t* out_tokens,
                         int32_t* num_out, int32_t* history, int64_t history_stride,
                         int32_t* history_len, int32_t* num_cached, const void* draft_logits,
                         int64_t ld_draft, const int32_t* draft_row_start, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(mode == NE_ACCEPT_GREEDY || mode == NE_ACCEPT_SAMPLED, "unknown mode %d", mode);
  NE_CHECK_ARG(vocab > 0, "vocab must be positive");
  NE_CHECK_ARG(drafts && num_drafts && row_start && out_tokens && num_out, "null pointer argument");
  NE_CHECK_ARG(max_drafts >= 1 && max_drafts < kMaxRows, "max_drafts must be in [1, %d]",
               kMaxRows - 1);
  if (mode == NE_ACCEPT_GREEDY) {
    NE_CHECK_ARG(logits || (argmax_partials && num_tiles > 0),
                 "greedy acceptance needs logits or argmax partials");
  } else {
    NE_CHECK_ARG(logits != nullptr, "sampled acceptance needs logits");
    NE_CHECK_ARG(temperature > 0.f, "sampled acceptance needs temperature > 0");
    NE_CHECK_ARG(seeds && steps, "sampled acceptance needs seeds and steps");
  }
  NE_CHECK_ARG(!logits || ld_logits >= vocab, "ld_logits < vocab");
  NE_CHECK_ARG(!history || (history_len && history_stride > 0), "history needs history_len");
  NE_CHECK_ARG(!draft_logits || (mode == NE_ACCEPT_SAMPLED && draft_row_start && ld_draft >= vocab),
               "draft rows need sampled mode, draft_row_start and ld_draft >= vocab");
  AcceptParams p{};
  p.mode = mode;
  p.logits = (const uint16_t*)logits;
  p.ld = ld_logits;
  p.partials = argmax_partials;
  p.num_tiles = num_tiles;
  p.vocab = vocab;
  p.drafts = drafts;
  p.max_drafts = max_drafts;
  p.num_drafts = num_drafts;
  p.row_start = row_start;
  p.temperature = temperature;
  p.seeds = seeds;
  p.steps = steps;
  p.out_tokens = out_tokens;
  p.num_out = num_out;
  p.history = history;
  p.hist_stride = history_stride;
  p.history_len = history_len;
  p.num_cached = num_cached;
  p.draft_logits = (const uint16_t*)draft_logits;
  p.dld = ld_draft;
  p.draft_row_start = draft_row_start;
  hipLaunchKernelGGL(accept_kernel, dim3(num_seqs), dim3(kThreads), 0, (hipStream_t)stream, p);
  return check_launch("accept");
}
