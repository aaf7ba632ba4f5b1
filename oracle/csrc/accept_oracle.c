/*
 * CPU oracle (test infrastructure only) for the acceptance step of the
 * speculative verify, under the explicit-uniform contract documented in
 * inference-engine-from-scratch_amd/csrc/accept.hip.
 *
 * Reference semantics restated: verify_proposal for a one-hot (n-gram) draft,
 * ne/engine/speculative/verifier.py:27-60; compute_token_probabilities,
 * ne/engine/sampling.py:30-38.  torch.rand / torch.multinomial draws are
 * replaced by Philox4x32-10 uniforms and an inverse CDF with a fixed summation
 * order, so this file and the GPU kernel must agree bit for bit.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -fno-fast-math -fPIC -shared
 * (oracle/Makefile).  No FMA contraction, so every operation below is a single
 * IEEE-754 binary32 operation.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define CHUNKS 256

/* Cephes expf (S. L. Moshier, Cephes Mathematical Library): Cody-Waite
 * reduction by ln 2 split in two constants, degree-5 polynomial for e^r - 1 - r.
 * Inputs below -86 return 0 so every result is a normal float. */
float oracle_cephes_exp(float x) {
  if (x < -86.0f) return 0.0f;
  float t = 1.44269504088896341f * x;
  t = t + 0.5f;
  const float fx = floorf(t);
  float r = x - fx * 0.693359375f;
  r = r - fx * -2.12194440e-4f;
  const float z = r * r;
  float y = 1.9875691500E-4f * r;
  y = y + 1.3981999507E-3f;
  y = y * r;
  y = y + 8.3334519073E-3f;
  y = y * r;
  y = y + 4.1665795894E-2f;
  y = y * r;
  y = y + 1.6666665459E-1f;
  y = y * r;
  y = y + 5.0000001201E-1f;
  y = y * z;
  y = y + r;
  y = y + 1.0f;
  const int n = (int)fx;
  uint32_t bits = (uint32_t)(n + 127) << 23;
  float scale;
  memcpy(&scale, &bits, sizeof(scale));
  return y * scale;
}

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11), rounds as in Random123. */
void oracle_philox4x32_10(uint32_t ctr[4], const uint32_t key[2]) {
  uint32_t k0 = key[0], k1 = key[1];
  for (int round = 0; round < 10; ++round) {
    if (round > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * ctr[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * ctr[2];
    const uint32_t out0 = (uint32_t)(p1 >> 32) ^ ctr[1] ^ k0;
    const uint32_t out1 = (uint32_t)p1;
    const uint32_t out2 = (uint32_t)(p0 >> 32) ^ ctr[3] ^ k1;
    const uint32_t out3 = (uint32_t)p0;
    ctr[0] = out0;
    ctr[1] = out1;
    ctr[2] = out2;
    ctr[3] = out3;
  }
}

float oracle_uniform(uint64_t seed, uint64_t step, int j) {
  uint32_t ctr[4] = {(uint32_t)step, (uint32_t)(step >> 32), (uint32_t)(j / 4), 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  oracle_philox4x32_10(ctr, key);
  return (float)(ctr[j % 4] >> 8) * (1.0f / 16777216.0f);
}

static float bf16_value(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, sizeof(f));
  return f;
}

/* e_j = exp(z_j - max z), z_j = logit_j / T, for one row */
static void row_exps(const uint16_t* row, int vocab, float temperature, float* e) {
  float mx = -INFINITY;
  for (int j = 0; j < vocab; ++j) {
    const float z = bf16_value(row[j]) / temperature;
    if (z > mx) mx = z;
  }
  for (int j = 0; j < vocab; ++j) e[j] = oracle_cephes_exp(bf16_value(row[j]) / temperature - mx);
}

/* sequential chunk sums of e with index `excl` removed (excl < 0: none) */
static void chunk_sums(const float* e, int vocab, int excl, float* sums) {
  const int ch = (vocab + CHUNKS - 1) / CHUNKS;
  for (int c = 0; c < CHUNKS; ++c) {
    float s = 0.0f;
    const int lo = c * ch;
    const int hi = lo + ch < vocab ? lo + ch : vocab;
    for (int j = lo; j < hi; ++j) s = s + (j == excl ? 0.0f : e[j]);
    sums[c] = s;
  }
}

static float total(const float* sums) {
  float z = 0.0f;
  for (int c = 0; c < CHUNKS; ++c) z = z + sums[c];
  return z;
}

/* inverse-CDF draw from e with `excl` removed; falls back to no exclusion when
 * the remaining mass is zero (verifier.py:54-56 uses p itself then) */
static int draw(const float* e, int vocab, int excl, float u) {
  const int ch = (vocab + CHUNKS - 1) / CHUNKS;
  float sums[CHUNKS];
  chunk_sums(e, vocab, excl, sums);
  float r = total(sums);
  if (!(r > 0.0f)) {
    excl = -1;
    chunk_sums(e, vocab, excl, sums);
    r = total(sums);
  }
  const float t = u * r;
  float prefix = 0.0f;
  for (int c = 0; c < CHUNKS; ++c) {
    if (prefix + sums[c] > t) {
      float q = 0.0f;
      const int lo = c * ch;
      const int hi = lo + ch < vocab ? lo + ch : vocab;
      for (int j = lo; j < hi; ++j) {
        q = q + (j == excl ? 0.0f : e[j]);
        if (prefix + q > t) return j;
      }
    }
    prefix = prefix + sums[c];
  }
  for (int j = vocab - 1; j >= 0; --j)
    if (j != excl && e[j] > 0.0f) return j;
  return 0;
}

/* ---- top-p (sampling.py:21-27) under the contract ----------------------------
 * Tokens rank by bf16 logit (larger first; -0 ranks as +0), ties by index.  With
 * M(v) = the chunked fp32 total of e_j over tokens whose key exceeds v, thr = top_p * Z:
 *   tau = the smallest key v with M(v) < thr (found by bisection over 16-bit keys);
 *   m   = the number of r in [0, H) with M(tau) + r * E(tau) < thr, H = tokens with
 *         key tau, E(tau) their common e value;
 *   a token is kept iff key > tau, or key == tau and fewer than m tokens of key tau
 *   precede it; K = chunked fp32 total of the kept e_j; p'_j = e_j / K when kept, else 0.
 * top_p >= 1 keeps every token (K = Z). */
static uint32_t key_of_bf16(uint16_t b) {
  if ((b & 0x7FFFu) == 0) b = 0;
  return (b & 0x8000u) ? (uint32_t)(~b & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}

static uint16_t bf16_of_key(uint32_t k) {
  return (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)(~k & 0xFFFFu);
}

typedef struct {
  const uint16_t* row; /* bf16 logits */
  int vocab;
  float temperature;
  float mx;
  float z;     /* chunked total of e */
  float total; /* K: chunked total of the kept e (z without top-p) */
  int topp;
  uint32_t tau;
  int m;
} row_dist;

static float dist_e(const row_dist* d, int j) {
  return oracle_cephes_exp(bf16_value(d->row[j]) / d->temperature - d->mx);
}

static float masked_total(const row_dist* d, uint32_t v) {
  const int ch = (d->vocab + CHUNKS - 1) / CHUNKS;
  float t = 0.0f;
  for (int c = 0; c < CHUNKS; ++c) {
    float s = 0.0f;
    const int lo = c * ch;
    const int hi = lo + ch < d->vocab ? lo + ch : d->vocab;
    for (int j = lo; j < hi; ++j)
      if (key_of_bf16(d->row[j]) > v) s = s + dist_e(d, j);
    t = t + s;
  }
  return t;
}

/* kept flags of a whole row in index order (the tie rank runs over the row) */
static void dist_kept(const row_dist* d, unsigned char* kept) {
  int ties = 0;
  for (int j = 0; j < d->vocab; ++j) {
    const uint32_t k = key_of_bf16(d->row[j]);
    if (!d->topp || k > d->tau) {
      kept[j] = 1;
    } else if (k == d->tau) {
      kept[j] = ties < d->m;
      ++ties;
    } else {
      kept[j] = 0;
    }
  }
}

static void dist_setup(row_dist* d, const uint16_t* row, int vocab, float temperature, float top_p,
                       unsigned char* kept, float* w) {
  d->row = row;
  d->vocab = vocab;
  d->temperature = temperature;
  float mx = -INFINITY;
  for (int j = 0; j < vocab; ++j) {
    const float zj = bf16_value(row[j]) / temperature;
    if (zj > mx) mx = zj;
  }
  d->mx = mx;
  for (int j = 0; j < vocab; ++j) w[j] = dist_e(d, j);
  float sums[CHUNKS];
  chunk_sums(w, vocab, -1, sums);
  d->z = total(sums);
  d->topp = top_p < 1.0f;
  d->tau = 0;
  d->m = 0;
  if (d->topp) {
    const float thr = top_p * d->z;
    uint32_t lo = 0, hi = 65535;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) / 2;
      if (masked_total(d, mid) < thr) hi = mid; else lo = mid + 1;
    }
    d->tau = lo;
    int h = 0;
    for (int j = 0; j < vocab; ++j) h += key_of_bf16(row[j]) == lo;
    const float mt = masked_total(d, lo);
    const float e_tau = oracle_cephes_exp(bf16_value(bf16_of_key(lo)) / temperature - mx);
    int a = 0, b = h; /* m = number of r in [0, h) with mt + r * e_tau < thr */
    while (a < b) {
      const int mid = (a + b) / 2;
      if (mt + (float)mid * e_tau < thr) a = mid + 1; else b = mid;
    }
    d->m = a;
  }
  dist_kept(d, kept);
  for (int j = 0; j < vocab; ++j) w[j] = kept[j] ? w[j] : 0.0f;
  chunk_sums(w, vocab, -1, sums);
  d->total = total(sums);
}

/*
 * Acceptance of one sequence under the contract with per-sequence top-p and an
 * optional draft distribution per guess:
 *   draft_rows == NULL     n-gram guesses (one-hot draft)
 *   draft_is_probs == 0    bf16 draft logits; q' = the same top-p softmax of the draft row
 *   draft_is_probs == 1    fp32 draft probabilities, used as given
 * Guess i is kept iff a >= 1 or (a > 0 and u_i < a), a = p'_g (one-hot) or
 * min(p'_g / max(q_g, 1e-12), 1); a rejection draws from p' without g (one-hot) or
 * from max(p' - q, 0) (each p'_j = e_j / K one fp32 division, each difference one op),
 * falling back to p' when that has no mass; the bonus draws from p'.
 * `scratch` holds 4 * vocab floats + 2 * vocab bytes.
 */
int oracle_accept_sampled_v2(const uint16_t* logits, int64_t ld, int vocab, const int32_t* drafts, int num_drafts,
                             float temperature, float top_p, const void* draft_rows, int draft_is_probs,
                             int64_t ldq, uint64_t seed, uint64_t step, int32_t* out, void* scratch) {
  float* w = (float*)scratch;
  float* f = w + vocab;
  float* r = f + vocab;
  unsigned char* kept = (unsigned char*)(r + vocab);
  unsigned char* keptq = kept + vocab;
  float sums[CHUNKS];
  int n_out = 0;
  for (int i = 0; i < num_drafts; ++i) {
    row_dist d;
    dist_setup(&d, logits + (int64_t)i * ld, vocab, temperature, top_p, kept, w);
    const int guess = drafts[i];
    const float p = kept[guess] ? w[guess] / d.total : 0.0f;
    const float u = oracle_uniform(seed, step, i);
    float a;
    row_dist dq;
    if (draft_rows == NULL) {
      a = p;
    } else if (draft_is_probs) {
      const float* q = (const float*)draft_rows + (int64_t)i * ldq;
      a = fminf(p / fmaxf(q[guess], 1e-12f), 1.0f);
    } else {
      dist_setup(&dq, (const uint16_t*)draft_rows + (int64_t)i * ldq, vocab, temperature, top_p, keptq, f);
      const float q = keptq[guess] ? f[guess] / dq.total : 0.0f;
      a = fminf(p / fmaxf(q, 1e-12f), 1.0f);
    }
    if (a >= 1.0f || (a > 0.0f && u < a)) {
      out[n_out++] = guess;
      continue;
    }
    const float u_draw = oracle_uniform(seed, step, 63);
    if (draft_rows == NULL) {
      out[n_out] = draw(w, vocab, guess, u_draw);
      return n_out + 1;
    }
    for (int j = 0; j < vocab; ++j) {
      const float pj = kept[j] ? w[j] / d.total : 0.0f;
      float qj;
      if (draft_is_probs) {
        qj = ((const float*)draft_rows)[(int64_t)i * ldq + j];
      } else {
        qj = keptq[j] ? f[j] / dq.total : 0.0f;
      }
      const float rj = pj - qj;
      r[j] = rj > 0.0f ? rj : 0.0f;
    }
    chunk_sums(r, vocab, -1, sums);
    out[n_out] = total(sums) > 0.0f ? draw(r, vocab, -1, u_draw) : draw(w, vocab, -1, u_draw);
    return n_out + 1;
  }
  row_dist d;
  dist_setup(&d, logits + (int64_t)num_drafts * ld, vocab, temperature, top_p, kept, w);
  out[n_out] = draw(w, vocab, -1, oracle_uniform(seed, step, 63));
  return n_out + 1;
}

/* kept flags and K of one row under top-p (for the pins) */
float oracle_top_p_kept(const uint16_t* row, int vocab, float temperature, float top_p, unsigned char* kept,
                        float* w, uint32_t* tau, int* m) {
  row_dist d;
  dist_setup(&d, row, vocab, temperature, top_p, kept, w);
  *tau = d.tau;
  *m = d.m;
  return d.total;
}

/*
 * One sequence: rows [num_drafts + 1][ld] bf16 logits (bit patterns), guesses
 * drafts[0..num_drafts).  Writes kept guesses + 1 token to out, returns the
 * count.  `scratch` holds vocab floats.
 */
int oracle_accept_sampled(const uint16_t* logits, int64_t ld, int vocab, const int32_t* drafts,
                          int num_drafts, float temperature, uint64_t seed, uint64_t step,
                          int32_t* out, float* scratch) {
  float sums[CHUNKS];
  int kept = 0;
  for (int i = 0; i < num_drafts; ++i) {
    const uint16_t* row = logits + (int64_t)i * ld;
    row_exps(row, vocab, temperature, scratch);
    chunk_sums(scratch, vocab, -1, sums);
    const float z = total(sums);
    const int guess = drafts[i];
    const float p = scratch[guess] / z;
    const float u = oracle_uniform(seed, step, i);
    if (p >= 1.0f || (p > 0.0f && u < p)) {
      out[kept++] = guess;
      continue;
    }
    out[kept] = draw(scratch, vocab, guess, oracle_uniform(seed, step, 63));
    return kept + 1;
  }
  row_exps(logits + (int64_t)num_drafts * ld, vocab, temperature, scratch);
  out[kept] = draw(scratch, vocab, -1, oracle_uniform(seed, step, 63));
  return kept + 1;
}

/*
 * oracle_accept_sampled with the guesses drawn by a draft model: draft rows
 * [num_drafts][ldq] hold the draft's logits for each guess (same temperature);
 * q = its softmax under the same contract.  Guess i is kept iff
 * a = min(p / max(q, 1e-12), 1) >= 1 or (a > 0 and u_i < a); a rejection draws
 * from r_j = max(p_j - q_j, 0) (p when r has no mass), verifier.py:36-56.
 * `scratch` holds 3 * vocab floats.
 */
int oracle_accept_sampled_draft(const uint16_t* logits, int64_t ld, const uint16_t* draft, int64_t ldq,
                                int vocab, const int32_t* drafts, int num_drafts, float temperature,
                                uint64_t seed, uint64_t step, int32_t* out, float* scratch) {
  float sums[CHUNKS];
  float* e = scratch;
  float* f = scratch + vocab;
  float* r = scratch + 2 * vocab;
  int kept = 0;
  for (int i = 0; i < num_drafts; ++i) {
    row_exps(logits + (int64_t)i * ld, vocab, temperature, e);
    chunk_sums(e, vocab, -1, sums);
    const float z = total(sums);
    row_exps(draft + (int64_t)i * ldq, vocab, temperature, f);
    chunk_sums(f, vocab, -1, sums);
    const float zq = total(sums);
    const int guess = drafts[i];
    const float p = e[guess] / z;
    const float q = fmaxf(f[guess] / zq, 1e-12f);
    const float a = fminf(p / q, 1.0f);
    const float u = oracle_uniform(seed, step, i);
    if (a >= 1.0f || (a > 0.0f && u < a)) {
      out[kept++] = guess;
      continue;
    }
    for (int j = 0; j < vocab; ++j) {
      const float rj = e[j] / z - f[j] / zq;
      r[j] = rj > 0.0f ? rj : 0.0f;
    }
    chunk_sums(r, vocab, -1, sums);
    const float u_draw = oracle_uniform(seed, step, 63);
    out[kept] = total(sums) > 0.0f ? draw(r, vocab, -1, u_draw) : draw(e, vocab, -1, u_draw);
    return kept + 1;
  }
  row_exps(logits + (int64_t)num_drafts * ld, vocab, temperature, e);
  out[kept] = draw(e, vocab, -1, oracle_uniform(seed, step, 63));
  return kept + 1;
}

/* ---- v3: integer masses for one-hot (n-gram) guesses -------------------------------
 * The contract the GPU's sampled n-gram path implements (csrc/accept.hip states it in
 * full).  Every token's weight is an integer that depends only on its bf16 key, so sums
 * in any order are exact and equal:
 *   invT = 1 / T (fp32 division); kmax = the row's largest key; mx = val(kmax) * invT;
 *   E(k) = (uint32)(exp3(val(k) * invT - mx) * 2^31), truncated; cnt(k) = tokens of key k;
 *   Z = sum cnt(k) E(k).  Top-p (P < 1): thr = max(1, (uint64)((double)Z * (double)P));
 *   M(v) = sum_{k > v} cnt(k) E(k); tau = the smallest v with M(v) < thr;
 *   m = min(cnt(tau), ceil((thr - M(tau)) / E(tau))); kept: key > tau, or key == tau
 *   and fewer than m tokens of key tau precede it; K = M(tau) + m E(tau).  P >= 1 keeps
 *   every token, K = Z.  w_j = E(key_j) when kept, else 0.
 *   Guess g of row i (U_i = the uniform's 24-bit integer) is kept iff w_g >= K or
 *   (w_g > 0 and U_i K < w_g 2^24).  A draw with x excluded (the rejected guess; none
 *   for the bonus): the kept tokens in order of key (descending) then index (ascending),
 *   x removed (kept if that leaves no weight); R = their total weight;
 *   t = floor(U R / 2^24); the token is the first whose running weight exceeds t.
 *   exp3: Cephes' Cody-Waite reduction and polynomial with each step one fused
 *   multiply-add (fmaf), 0 below -86. */
float oracle_exp3(float x) {
  if (x < -86.0f) return 0.0f;
  const float fx = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
  float r = fmaf(fx, -0.693359375f, x);
  r = fmaf(fx, 2.12194440e-4f, r);
  float y = fmaf(1.9875691500E-4f, r, 1.3981999507E-3f);
  y = fmaf(y, r, 8.3334519073E-3f);
  y = fmaf(y, r, 4.1665795894E-2f);
  y = fmaf(y, r, 1.6666665459E-1f);
  y = fmaf(y, r, 5.0000001201E-1f);
  const float z = r * r;
  y = fmaf(y, z, r);
  y = y + 1.0f;
  const int n = (int)fx;
  uint32_t bits = (uint32_t)(n + 127) << 23;
  float scale;
  memcpy(&scale, &bits, sizeof(scale));
  return y * scale;
}

typedef struct {
  uint32_t cnt[65536];
  int vocab;
  uint32_t kmax;
  float invT, mx;
  uint64_t z, k_total, thr;
  int topp;
  uint32_t tau, m;
} v3_row;

static uint32_t v3_weight(const v3_row* d, uint32_t k) {
  const float e = oracle_exp3(bf16_value(bf16_of_key(k)) * d->invT - d->mx);
  return (uint32_t)(e * 2147483648.0f);
}

static void v3_setup(v3_row* d, const uint16_t* row, int vocab, float temperature, float top_p) {
  memset(d->cnt, 0, sizeof(d->cnt));
  d->vocab = vocab;
  d->kmax = 0;
  for (int j = 0; j < vocab; ++j) {
    const uint32_t k = key_of_bf16(row[j]);
    d->cnt[k] += 1;
    if (k > d->kmax) d->kmax = k;
  }
  d->invT = 1.0f / temperature;
  d->mx = bf16_value(bf16_of_key(d->kmax)) * d->invT;
  uint64_t z = 0;
  for (uint32_t k = 0; k < 65536; ++k)
    if (d->cnt[k]) z += (uint64_t)d->cnt[k] * v3_weight(d, k);
  d->z = z;
  d->topp = top_p < 1.0f;
  d->tau = 0;
  d->m = 0;
  d->k_total = z;
  d->thr = 0;
  if (!d->topp) return;
  uint64_t thr = (uint64_t)((double)z * (double)top_p);
  if (thr < 1) thr = 1;
  d->thr = thr;
  uint64_t above = 0; /* M(k) while walking down */
  for (int k = 65535; k >= 0; --k) {
    const uint64_t mass = d->cnt[k] ? (uint64_t)d->cnt[k] * v3_weight(d, (uint32_t)k) : 0;
    if (above + mass >= thr) { /* M(k) = above < thr <= M(k - 1) */
      const uint64_t e = v3_weight(d, (uint32_t)k);
      uint64_t m = (thr - above + e - 1) / e;
      if (m > d->cnt[k]) m = d->cnt[k];
      d->tau = (uint32_t)k;
      d->m = (uint32_t)m;
      d->k_total = above + m * e;
      return;
    }
    above += mass;
  }
}

/* kept (1) or not (0) for token j of the row */
static int v3_kept(const v3_row* d, const uint16_t* row, int j) {
  if (j < 0 || j >= d->vocab) return 0; /* a guess outside the vocabulary weighs 0 */
  const uint32_t k = key_of_bf16(row[j]);
  if (!d->topp || k > d->tau) return 1;
  if (k < d->tau) return 0;
  uint32_t rank = 0;
  for (int i = 0; i < j; ++i) rank += key_of_bf16(row[i]) == d->tau;
  return rank < d->m;
}

/* floor(u * r / 2^24) for u < 2^24, exactly */
static uint64_t v3_scale(uint32_t u, uint64_t r) {
  return (uint64_t)u * (r >> 24) + (((uint64_t)u * (r & 0xFFFFFFu)) >> 24);
}

static int v3_draw(const v3_row* d, const uint16_t* row, int vocab, int x, uint32_t u) {
  uint64_t wx = 0;
  if (x >= 0 && v3_kept(d, row, x)) wx = v3_weight(d, key_of_bf16(row[x]));
  if (x >= vocab) x = -1;
  uint64_t r = d->k_total - wx;
  if (r == 0) { /* x held all the kept weight: draw without the exclusion */
    x = -1;
    wx = 0;
    r = d->k_total;
  }
  const uint64_t t = v3_scale(u, r);
  const uint32_t kx = x >= 0 ? key_of_bf16(row[x]) : 0xFFFFFFFFu;
  uint64_t run = 0;
  for (int k = (int)d->kmax; k >= 0; --k) {
    uint64_t c = d->cnt[k];
    if (d->topp && (uint32_t)k < d->tau) break;
    if (d->topp && (uint32_t)k == d->tau) c = d->m;
    if (wx && (uint32_t)k == kx) c -= 1;
    if (!c) continue;
    const uint64_t e = v3_weight(d, (uint32_t)k);
    if (!e) continue;
    if (run + c * e > t) {
      const uint64_t want = (t - run) / e; /* the want-th kept occurrence of k, x skipped */
      uint64_t seen = 0;
      for (int j = 0; j < vocab; ++j) {
        if (key_of_bf16(row[j]) != (uint32_t)k || j == x) continue;
        if (seen == want) return j;
        ++seen;
      }
      return -1; /* unreachable */
    }
    run += c * e;
  }
  return -1; /* unreachable: t < r */
}

/*
 * One sequence under v3: rows [num_drafts + 1][ld] bf16 logit bit patterns, guesses
 * drafts[0..num_drafts).  Writes kept guesses + 1 token to out and returns the count.
 * `scratch` holds sizeof(v3_row) bytes (oracle_v3_scratch_bytes()).
 */
int oracle_accept_sampled_v3(const uint16_t* logits, int64_t ld, int vocab, const int32_t* drafts, int num_drafts,
                             float temperature, float top_p, uint64_t seed, uint64_t step, int32_t* out,
                             void* scratch) {
  v3_row* d = (v3_row*)scratch;
  int n_out = 0;
  for (int i = 0; i <= num_drafts; ++i) {
    const uint16_t* row = logits + (int64_t)i * ld;
    v3_setup(d, row, vocab, temperature, top_p);
    const float u_draw = oracle_uniform(seed, step, 63);
    const uint32_t ud = (uint32_t)(u_draw * 16777216.0f);
    if (i == num_drafts) {
      out[n_out] = v3_draw(d, row, vocab, -1, ud);
      return n_out + 1;
    }
    const int guess = drafts[i];
    const uint64_t w = v3_kept(d, row, guess) ? v3_weight(d, key_of_bf16(row[guess])) : 0; /* 0 when outside */
    const uint32_t ui = (uint32_t)(oracle_uniform(seed, step, i) * 16777216.0f);
    const int accept = w >= d->k_total || (w > 0 && (unsigned __int128)ui * d->k_total < (unsigned __int128)w << 24);
    if (accept) {
      out[n_out++] = guess;
      continue;
    }
    out[n_out] = v3_draw(d, row, vocab, guess, ud);
    return n_out + 1;
  }
  return n_out; /* unreachable */
}

size_t oracle_v3_scratch_bytes(void) { return sizeof(v3_row); }

/* the v3 kept flags, K, Z, tau and m of one row (for the pins) */
uint64_t oracle_v3_row(const uint16_t* row, int vocab, float temperature, float top_p, unsigned char* kept,
                       uint64_t* z, uint32_t* tau, uint32_t* m, void* scratch) {
  v3_row* d = (v3_row*)scratch;
  v3_setup(d, row, vocab, temperature, top_p);
  uint32_t ties = 0;
  for (int j = 0; j < vocab; ++j) {
    const uint32_t k = key_of_bf16(row[j]);
    if (!d->topp || k > d->tau) {
      kept[j] = 1;
    } else if (k == d->tau) {
      kept[j] = ties < d->m;
      ++ties;
    } else {
      kept[j] = 0;
    }
  }
  *z = d->z;
  *tau = d->tau;
  *m = d->m;
  return d->k_total;
}

/* E(k) of a row (for the pins): the weight of a token with key k */
uint32_t oracle_v3_weight(const uint16_t* row, int vocab, float temperature, uint32_t key, void* scratch) {
  v3_row* d = (v3_row*)scratch;
  v3_setup(d, row, vocab, temperature, 1.0f);
  return v3_weight(d, key);
}
