// n-gram prompt-lookup drafting on the device token history (gfx950).
//
// Restates NgramProposer.propose (ne/engine/speculative/proposers.py:44-57) for a
// batch: one 256-thread work-group per sequence.  For each n (max_ngram down to
// min_ngram, skipping n >= len) the reference scans starts from len-n-1 downward and
// returns the first window equal to the last n tokens.  A window of length n starting
// at s ends at e = s + n - 1 <= len - 2, and it matches exactly when the tokens ending
// at e and those ending at len - 1 agree on their last n; so one pass over end
// positions e = len - 2, len - 3, ..., computing that agreement length c(e) (up to
// max_ngram), finds for every n the largest matching e at once.  The pass runs 4096
// ends at a time (16 per thread) against the chunk's stretch of history, staged in LDS
// with one coalesced load, and stops after the first chunk holding a max_ngram match,
// which is the common case in long histories; without one, the same pass has already
// found the smaller n's answers.  The guesses are the tokens that followed
// the window, clipped to the history, so they are never empty.
#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kMaxNgram = 16;
constexpr int kScanPerThread = 16;
constexpr int kScanChunk = 256 * kScanPerThread;  // ends per pass
constexpr int kStage = kScanChunk + kMaxNgram;     // history tokens a pass compares

// The counters a verify step leaves for the next one (adv != nullptr): the work-group of
// sequence b first advances b's counters and takes its guess count from them.
struct StepCounters {
  const int32_t* num_out;
  const int32_t* max_new;
  int32_t* generated;
  uint64_t* steps;
  int32_t* num_guesses;
  int k;
};

__global__ __launch_bounds__(256) void ngram_kernel(const int32_t* history, int64_t stride,
                                                    const int32_t* history_len,
                                                    const int32_t* num_tokens, int max_ngram,
                                                    int min_ngram, int max_drafts, int32_t* drafts,
                                                    int32_t* num_drafts, StepCounters adv) {
  __shared__ int s_best[kMaxNgram][256 / kWave];
  __shared__ int s_hist[kStage];
  __shared__ int s_want;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t* h = history + (int64_t)b * stride;
  const int len = history_len[b];
  int requested = 0;
  if (adv.num_out != nullptr) {
    // ne_advance_step_counts for slot b, by one thread, whose loads go out with the
    // length's; the others take its count after the scan's first barrier (or the one
    // below when there is no scan), so none reads a counter after it was advanced
    if (tid == 0) {
      const int gen0 = adv.generated[b], out = adv.num_out[b], cap = adv.max_new[b];
      const uint64_t steps = adv.steps[b];
      int g = 0;
      if (len > 0) {
        const int gen = gen0 + out;
        adv.generated[b] = gen;
        adv.steps[b] = steps + 1;
        g = max(0, min(adv.k, cap - gen - 1));
      }
      adv.num_guesses[b] = g;
      s_want = g;
    }
  } else {
    requested = num_tokens[b];
  }
  const int nmax = min(max_ngram, len - 1);  // n < len
  // the scan does not depend on the guess count, so with the step counters it starts
  // before the count is known and stops after its first chunk when the count is 0; a
  // count passed in (num_tokens, read by every thread) of 0 skips it
  const bool scan = nmax >= min_ngram && (adv.num_out != nullptr || requested > 0);  // uniform
  int suffix[kMaxNgram];  // the history read backwards from its last token
#pragma unroll
  for (int i = 0; i < kMaxNgram; ++i) suffix[i] = (i < nmax) ? h[len - 1 - i] : 0;
  int found[kMaxNgram];  // found[n - 1]: the largest end e of an n-window match so far
#pragma unroll
  for (int i = 0; i < kMaxNgram; ++i) found[i] = -1;
  if (!scan) __syncthreads();  // uniform: publishes s_want
  for (int hi = scan ? len - 2 : -1; hi >= 0; hi -= kScanChunk) {
    // the pass's ends are hi - 4095 .. hi and their windows reach 15 tokens further back:
    // s_hist[k] = h[base + k] for the history positions 0 .. hi among them.  The previous
    // pass's reads of s_hist ended before its last barrier.
    const int base = hi - kScanChunk - kMaxNgram + 2;
    for (int k = tid; k < kStage; k += 256) {
      const int pos = base + k;
      s_hist[k] = (pos >= 0 && pos <= hi) ? h[pos] : 0;
    }
    __syncthreads();
    // thread tid tests ends hi - tid, hi - tid - 256, ...: its first hit for each n is
    // its largest, and the owner of the chunk's largest hit has no larger one
    int best[kMaxNgram];
#pragma unroll
    for (int i = 0; i < kMaxNgram; ++i) best[i] = -1;
    // the last token of each of this thread's ends first: only an end that matches it
    // reads the rest of its window (most do not), in the same order, largest end first
    uint32_t hit = 0;
#pragma unroll
    for (int j = 0; j < kScanPerThread; ++j) {
      const int e = hi - j * 256 - tid;
      if (e >= 0 && s_hist[e - base] == suffix[0]) hit |= 1u << j;
    }
    while (hit != 0) {
      const int j = __builtin_ctz(hit);
      hit &= hit - 1;
      const int e = hi - j * 256 - tid;
      // the window's tokens are all read before the first comparison, so the LDS reads
      // overlap (e - i - base >= 0 for every i: the stage reaches 15 tokens below the
      // pass's lowest end)
      int tok[kMaxNgram];
#pragma unroll
      for (int i = 0; i < kMaxNgram; ++i) tok[i] = s_hist[e - i - base];
      int c = 0;  // tokens ending at e that equal those ending at len - 1
      bool same = true;
#pragma unroll
      for (int i = 0; i < kMaxNgram; ++i) {
        if (same && i < nmax && e - i >= 0 && tok[i] == suffix[i]) {
          ++c;
        } else {
          same = false;
        }
      }
#pragma unroll
      for (int i = 0; i < kMaxNgram; ++i)
        if (i < c && best[i] < 0) best[i] = e;
    }
#pragma unroll
    for (int i = 0; i < kMaxNgram; ++i) {
      if (i + 1 >= min_ngram && i < nmax) {  // uniform
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) best[i] = max(best[i], __shfl_xor(best[i], o));
        if (tid % kWave == 0) s_best[i][tid / kWave] = best[i];
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kMaxNgram; ++i) {
      if (i + 1 >= min_ngram && i < nmax) {
        int top = s_best[i][0];
#pragma unroll
        for (int w = 1; w < 256 / kWave; ++w) top = max(top, s_best[i][w]);
        if (found[i] < 0) found[i] = top;
      }
    }
    __syncthreads();
    bool done = false;
#pragma unroll
    for (int i = 0; i < kMaxNgram; ++i)
      if (i == nmax - 1) done = found[i] >= 0;
    if (done) break;  // uniform: the largest n has its answer
    if (adv.num_out != nullptr && s_want <= 0) break;  // uniform: published before the barriers above
  }
  if (adv.num_out != nullptr) requested = s_want;
  const int want = min(requested, max_drafts);
  if (want <= 0 || !scan) {
    if (tid == 0) num_drafts[b] = 0;
    return;
  }
  // the largest n with a match
  int e = -1;
#pragma unroll
  for (int i = 0; i < kMaxNgram; ++i)
    if (i + 1 >= min_ngram && i < nmax && found[i] >= 0) e = found[i];
  if (e < 0) {
    if (tid == 0) num_drafts[b] = 0;
    return;
  }
  const int follow = e + 1;
  const int count = min(want, len - follow);
  for (int i = tid; i < count; i += 256) drafts[(int64_t)b * max_drafts + i] = h[follow + i];
  if (tid == 0) num_drafts[b] = count;
}

}  // namespace

}  // namespace ne

using namespace ne;

extern "C" int ne_ngram_propose(const int32_t* history, int64_t history_stride,
                                const int32_t* history_len, const int32_t* num_tokens,
                                int32_t num_seqs, int32_t max_ngram, int32_t min_ngram,
                                int32_t max_drafts, int32_t* drafts, int32_t* num_drafts,
                                void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(history && history_len && num_tokens && drafts && num_drafts,
               "null pointer argument");
  NE_CHECK_ARG(min_ngram >= 1 && max_ngram >= min_ngram, "need 1 <= min_ngram <= max_ngram");
  NE_CHECK_SUPPORTED(max_ngram <= kMaxNgram, "max_ngram must be <= %d (got %d)", kMaxNgram,
                     max_ngram);
  NE_CHECK_ARG(max_drafts >= 1, "max_drafts must be >= 1");
  NE_CHECK_ARG(history_stride >= 1, "history_stride must be >= 1");
  hipLaunchKernelGGL(ngram_kernel, dim3(num_seqs), dim3(256), 0, (hipStream_t)stream, history,
                     history_stride, history_len, num_tokens, max_ngram, min_ngram, max_drafts,
                     drafts, num_drafts, StepCounters{});
  return check_launch("ngram_propose");
}

extern "C" int ne_advance_and_propose(const int32_t* history, int64_t history_stride,
                                      const int32_t* history_len, const int32_t* num_out,
                                      const int32_t* max_new_tokens, int32_t* num_generated,
                                      uint64_t* steps, int32_t* num_guesses, int32_t k, int32_t num_seqs,
                                      int32_t max_ngram, int32_t min_ngram, int32_t max_drafts,
                                      int32_t* drafts, int32_t* num_drafts, void* stream) {
  NE_CHECK_ARG(num_seqs >= 0 && k >= 0, "bad sizes (num_seqs=%d, k=%d)", num_seqs, k);
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(history && history_len && num_out && max_new_tokens && num_generated && steps && num_guesses &&
                   drafts && num_drafts,
               "null pointer argument");
  NE_CHECK_ARG(min_ngram >= 1 && max_ngram >= min_ngram, "need 1 <= min_ngram <= max_ngram");
  NE_CHECK_SUPPORTED(max_ngram <= kMaxNgram, "max_ngram must be <= %d (got %d)", kMaxNgram,
                     max_ngram);
  NE_CHECK_ARG(max_drafts >= 1, "max_drafts must be >= 1");
  NE_CHECK_ARG(history_stride >= 1, "history_stride must be >= 1");
  const StepCounters adv{num_out, max_new_tokens, num_generated, steps, num_guesses, k};
  hipLaunchKernelGGL(ngram_kernel, dim3(num_seqs), dim3(256), 0, (hipStream_t)stream, history,
                     history_stride, history_len, num_guesses, max_ngram, min_ngram, max_drafts,
                     drafts, num_drafts, adv);
  return check_launch("advance_and_propose");
}
