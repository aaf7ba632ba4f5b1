// n-gram prompt-lookup drafting on the device token history (gfx950).
//
// Restates NgramProposer.propose (ne/engine/speculative/proposers.py:44-57) for a
// batch: one 256-thread work-group per sequence.  For n = max_ngram..min_ngram
// (skipping n >= len) the work-group tests start positions from len-n-1 downward,
// 1024 at a time (4 per thread), and stops after the first chunk holding a start
// whose window equals the last n tokens, keeping the largest such start -- the
// reference scans starts from len-n-1 downward and returns the first match, which
// is the same window.  A recent match (the common case in long histories) costs one
// chunk instead of a scan of the whole history.  The guesses are the tokens that
// followed it, clipped to the history, so they are never empty.
#include "ne_common.hpp"

namespace ne {

namespace {

constexpr int kMaxNgram = 16;
constexpr int kScanPerThread = 4;
constexpr int kScanChunk = 256 * kScanPerThread;

__global__ __launch_bounds__(256) void ngram_kernel(const int32_t* history, int64_t stride,
                                                    const int32_t* history_len,
                                                    const int32_t* num_tokens, int max_ngram,
                                                    int min_ngram, int max_drafts, int32_t* drafts,
                                                    int32_t* num_drafts) {
  __shared__ int s_best[256 / kWave];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t* h = history + (int64_t)b * stride;
  const int len = history_len[b];
  const int want = min(num_tokens[b], max_drafts);
  if (want <= 0) {
    if (tid == 0) num_drafts[b] = 0;
    return;
  }
  for (int n = max_ngram; n >= min_ngram; --n) {
    if (len <= n) continue;
    int suffix[kMaxNgram];
#pragma unroll
    for (int i = 0; i < kMaxNgram; ++i) suffix[i] = (i < n) ? h[len - n + i] : 0;
    int top = -1;
    for (int hi = len - n - 1; hi >= 0 && top < 0; hi -= kScanChunk) {
      // thread tid tests starts hi - tid, hi - tid - 256, ...: its first hit is its
      // largest, and the owner of the chunk's largest hit has no larger one
      int best = -1;
#pragma unroll
      for (int j = 0; j < kScanPerThread; ++j) {
        const int start = hi - j * 256 - tid;
        if (start >= 0 && best < 0) {
          bool eq = true;
#pragma unroll
          for (int i = 0; i < kMaxNgram; ++i)
            if (i < n) eq = eq && (h[start + i] == suffix[i]);
          if (eq) best = start;
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) best = max(best, __shfl_xor(best, o));
      if (tid % kWave == 0) s_best[tid / kWave] = best;
      __syncthreads();
      top = s_best[0];
#pragma unroll
      for (int w = 1; w < 256 / kWave; ++w) top = max(top, s_best[w]);
      __syncthreads();
    }
    if (top >= 0) {
      const int follow = top + n;
      const int count = min(want, len - follow);
      for (int i = tid; i < count; i += 256) drafts[(int64_t)b * max_drafts + i] = h[follow + i];
      if (tid == 0) num_drafts[b] = count;
      return;
    }
  }
  if (tid == 0) num_drafts[b] = 0;
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
                     drafts, num_drafts);
  return check_launch("ngram_propose");
}
