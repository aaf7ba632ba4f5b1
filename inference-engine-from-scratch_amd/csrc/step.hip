// Device-side packing of one batched verify step (gfx950).
//
// Replaces build_step_inputs for the verify step
// (ne/engine/generation/batch_builder.py:22-65, paged_allocator.py:69-79):
// sequence b gets rows b*R .. b*R+R-1 with R = max_drafts + 1.  Row i <= g_b
// holds the last accepted token (i = 0) or guess i-1, at position L_b - 1 + i
// (L_b = history length, all but the last token cached); its key/value slot is
// block_tables[b, pos / bs] * bs + pos % bs.  Rows past the sequence's guesses
// are padding: token 0, position 0, the scratch slot, as the reference pads.
// A sequence with history_len 0 is inactive (q_len 0: no attention, all pads).
#include "ne_common.hpp"

namespace ne {
namespace {

__global__ __launch_bounds__(256) void prepare_verify_kernel(
    const int32_t* history, int64_t hist_stride, const int32_t* history_len, const int32_t* drafts,
    int max_drafts, const int32_t* num_drafts, const int32_t* block_tables, int bt_stride,
    int block_size, int scratch_slot, int num_seqs, int32_t* tokens, int32_t* positions,
    int32_t* slot_mapping, int32_t* q_start, int32_t* q_len, int32_t* ctx_len) {
  const int R = max_drafts + 1;
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= num_seqs * R) return;
  const int b = row / R;
  const int i = row % R;
  const int L = history_len[b];
  // a count outside [0, max_drafts] would read past the sequence's rows and table
  const int g = (L > 0) ? min(max(num_drafts[b], 0), max_drafts) : -1;
  if (i <= g) {
    const int pos = L - 1 + i;
    tokens[row] = (i == 0) ? history[(int64_t)b * hist_stride + L - 1]
                           : drafts[(int64_t)b * max_drafts + i - 1];
    positions[row] = pos;
    const int blk = block_tables[(int64_t)b * bt_stride + pos / block_size];
    slot_mapping[row] = blk * block_size + pos % block_size;
  } else {
    tokens[row] = 0;
    positions[row] = 0;
    slot_mapping[row] = scratch_slot;
  }
  if (i == 0) {
    q_start[b] = b * R;
    q_len[b] = g + 1;
    ctx_len[b] = (L > 0) ? L + g : 0;
  }
}

// After a verify step, per sequence b: when active (history_len > 0) add the tokens it
// emitted to its generated count, advance its sampling step and set the next step's
// guess count min(k, max_new - generated - 1) clipped at 0
// (speculative_generator.py:71-72, the rule of num_guesses); inactive: 0 guesses.
__global__ __launch_bounds__(256) void advance_counts_kernel(const int32_t* history_len,
                                                             const int32_t* num_out,
                                                             const int32_t* max_new, int32_t* generated,
                                                             uint64_t* steps, int32_t* num_guesses, int k,
                                                             int num_seqs) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= num_seqs) return;
  if (history_len[b] <= 0) {
    num_guesses[b] = 0;
    return;
  }
  const int gen = generated[b] + num_out[b];
  generated[b] = gen;
  steps[b] += 1;
  num_guesses[b] = max(0, min(k, max_new[b] - gen - 1));
}

}  // namespace
}  // namespace ne

using namespace ne;

extern "C" int ne_advance_step_counts(const int32_t* history_len, const int32_t* num_out,
                                      const int32_t* max_new_tokens, int32_t* num_generated,
                                      uint64_t* steps, int32_t* num_guesses, int32_t k, int32_t num_seqs,
                                      void* stream) {
  NE_CHECK_ARG(num_seqs >= 0 && k >= 0, "bad sizes (num_seqs=%d, k=%d)", num_seqs, k);
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(history_len && num_out && max_new_tokens && num_generated && steps && num_guesses,
               "null pointer argument");
  hipLaunchKernelGGL(advance_counts_kernel, dim3(ceil_div(num_seqs, 256)), dim3(256), 0, (hipStream_t)stream,
                     history_len, num_out, max_new_tokens, num_generated, steps, num_guesses, k, num_seqs);
  return check_launch("advance_step_counts");
}

extern "C" int ne_prepare_verify_step(const int32_t* history, int64_t history_stride,
                                      const int32_t* history_len, const int32_t* drafts,
                                      int32_t max_drafts, const int32_t* num_drafts,
                                      const int32_t* block_tables, int32_t block_table_stride,
                                      int32_t block_size, int32_t scratch_slot, int32_t num_seqs,
                                      int32_t* tokens, int32_t* positions, int32_t* slot_mapping,
                                      int32_t* q_start, int32_t* q_len, int32_t* ctx_len,
                                      void* stream) {
  NE_CHECK_ARG(num_seqs >= 0, "num_seqs < 0");
  if (num_seqs == 0) return NE_OK;
  NE_CHECK_ARG(history && history_len && drafts && num_drafts && block_tables && tokens &&
                   positions && slot_mapping && q_start && q_len && ctx_len,
               "null pointer argument");
  NE_CHECK_ARG(max_drafts >= 1 && block_size >= 1 && scratch_slot >= 0, "bad sizes");
  const int rows = num_seqs * (max_drafts + 1);
  hipLaunchKernelGGL(prepare_verify_kernel, dim3(ceil_div(rows, 256)), dim3(256), 0,
                     (hipStream_t)stream, history, history_stride, history_len, drafts, max_drafts,
                     num_drafts, block_tables, block_table_stride, block_size, scratch_slot,
                     num_seqs, tokens, positions, slot_mapping, q_start, q_len, ctx_len);
  return check_launch("prepare_verify_step");
}
