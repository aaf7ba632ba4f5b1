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
