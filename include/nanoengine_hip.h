/*
 * nanoengine_hip.h - C ABI of libnanoengine_hip.so, the gfx950 (MI355X) kernels
 * behind nanoengine's speculative-decoding verify step.
 *
 * Every entry point takes raw device pointers, plain integer sizes/strides, a
 * dtype enum and the hipStream_t to launch on (passed as void* so this header
 * needs no HIP include).  Nothing here allocates, frees or synchronises; a
 * caller-owned workspace is passed where a kernel needs scratch memory.  All
 * launches are asynchronous on `stream`.
 *
 * Return value: NE_OK (0) or a negative NE_E* code; ne_last_error() then gives a
 * message for the calling thread.  Shapes are validated on the host before any
 * launch, so an invalid call launches nothing.
 *
 * Reference interfaces each entry point replaces are cited as
 * path:line relative to the reference tree, with
 *   ne/ = nanoengine/src/nanoengine/
 */
#ifndef NANOENGINE_HIP_H
#define NANOENGINE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NE_ABI_VERSION 10

/* status codes */
#define NE_OK 0
#define NE_EINVAL (-1)       /* bad argument (shape, dtype, null pointer, size) */
#define NE_EUNSUPPORTED (-2) /* valid but not implemented (e.g. head_dim != 128) */
#define NE_ELAUNCH (-3)      /* hipLaunchKernel / hipGetLastError reported an error */
#define NE_EWORKSPACE (-4)   /* workspace too small: query the *_workspace_size call */

/* element types */
#define NE_DTYPE_BF16 0
#define NE_DTYPE_FP16 1
#define NE_DTYPE_FP32 2
#define NE_DTYPE_INT8 3

/* GEMM epilogues */
#define NE_EPILOGUE_STORE 0  /* y = bf16(acc * scale[n]) */
#define NE_EPILOGUE_SWIGLU 1 /* y[:, j] = bf16(silu(gate_j) * up_j), weight rows paired per 16 */

int ne_abi_version(void);
const char* ne_last_error(void);

/*
 * A1 - n-gram prompt-lookup drafting (replaces NgramProposer.propose,
 * ne/engine/speculative/proposers.py:39-57, one sequence per call there).
 * For each sequence b: for n = max_ngram..min_ngram, skip when len <= n; the
 * suffix is the last n tokens; scan start = len-n-1 down to 0 and take the first
 * window equal to the suffix; drafts = history[start+n : start+n+num_tokens[b]]
 * (clipped to len, never empty).  No match or num_tokens[b] == 0 gives 0 drafts.
 *   history      [num_seqs, history_stride] int32, history_len[b] valid tokens
 *   num_tokens   [num_seqs] int32, guesses requested (<= max_drafts)
 *   drafts       [num_seqs, max_drafts] int32 out (unused tail untouched)
 *   num_drafts   [num_seqs] int32 out
 */
int ne_ngram_propose(const int32_t* history, int64_t history_stride, const int32_t* history_len,
                     const int32_t* num_tokens, int32_t num_seqs, int32_t max_ngram,
                     int32_t min_ngram, int32_t max_drafts, int32_t* drafts, int32_t* num_drafts,
                     void* stream);

/*
 * A7 - quantise-and-scatter new key or value vectors into one layer's slot pool
 * (replaces write_to_cache + quantize_vectors, ne/models/attention_context.py:42-54,
 * ne/models/int8_quantization.py:30-34).
 *   vectors      [n, num_heads, head_dim] bf16 or fp16 (vec_dtype), contiguous
 *   slot_mapping [n] int32 target slot per vector row
 *   cache        [num_slots+1, num_heads, head_dim], int8 when cache_dtype is
 *                NE_DTYPE_INT8, else vec_dtype (plain scatter)
 *   scales       [num_slots+1, num_heads] in scale_dtype (int8 cache only)
 * int8: s = max(max|x|, 1e-8) / 127 in fp32 (IEEE division); q = rint(x / s)
 * clamped to [-127, 127]; the stored scale is s rounded to scale_dtype.
 */
int ne_kv_write(const void* vectors, int32_t vec_dtype, int64_t n, int32_t num_heads,
                int32_t head_dim, const int32_t* slot_mapping, void* cache, int32_t cache_dtype,
                void* scales, int32_t scale_dtype, void* stream);

/*
 * A6 - paged multi-query verify attention over a slot pool read in place
 * (replaces read_from_cache + scaled_dot_product_attention in
 * run_cached_attention, ne/models/attention_context.py:57-109, and the padded
 * context-slot / mask construction of ne/engine/generation/batch_builder.py:22-65
 * and ne/engine/memory/paged_allocator.py:69-79).
 * Sequence b owns query rows q_start[b] .. q_start[b]+q_len[b]-1 of q/out; its
 * context is ctx_len[b] tokens (cached tokens plus this step's q_len[b]); the
 * query at row i sits at position ctx_len[b]-q_len[b]+i and sees keys 0..pos.
 * Key position p lives in slot block_tables[b, p / block_size] * block_size +
 * p % block_size.  Query head h uses KV head h / (num_q_heads / num_kv_heads).
 *   q, out       bf16, element (row, head, d) at row*token_stride + head*head_stride + d
 *   k/v_cache    [num_slots+1, num_kv_heads, 128] bf16 or int8 (kv_dtype)
 *   k/v_scale    [num_slots+1, num_kv_heads] bf16 or fp16 (int8 cache only)
 *   workspace    ne_paged_attention_workspace_size() bytes.  Bytes 0..3 hold an
 *                error flag, set non-zero when a sequence's context exceeded
 *                max_ctx_len (its keys past max_ctx_len, or past the split grid,
 *                are then dropped); the caller clears it.  The rest holds the work
 *                plan and fp32 split partials, written and consumed within the
 *                call (no state carries between calls).
 * split_len: most keys per work-group (multiple of 128 up to 2048; 0 = choose: the
 * int8 / 8-KV-head path then sizes each sequence's splits from the total work, at
 * least 256 keys each).  head_dim must be 128 and block_size a multiple of 16.  One
 * work-group serves every KV head of a sequence's split; splits are combined by a
 * second kernel on the same stream.
 */
size_t ne_paged_attention_workspace_size(int32_t num_seqs, int32_t num_q_heads,
                                         int32_t num_kv_heads, int32_t max_q_len,
                                         int32_t max_ctx_len, int32_t split_len);
int ne_paged_verify_attention(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                              const void* k_cache, const void* v_cache, const void* k_scale,
                              const void* v_scale, int32_t kv_dtype, int32_t scale_dtype,
                              const int32_t* block_tables, int32_t block_table_stride,
                              int32_t block_size, const int32_t* ctx_len, const int32_t* q_start,
                              const int32_t* q_len, int32_t num_seqs, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim, int32_t max_q_len,
                              int32_t max_ctx_len, float softmax_scale, void* out,
                              int64_t out_token_stride, int64_t out_head_stride, int32_t split_len,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of ne_paged_verify_attention (no counterpart in the reference:
 * for callers that cannot allocate or pass a workspace -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The same arguments and the same
 * results as ne_paged_verify_attention, except that the work plan and split partials live
 * in a library-owned device array of NE_NOALLOC_SCRATCH_BYTES per GPU (held until the
 * process ends), and the error flag is the caller's device word `error_flag` (bits are
 * OR-ed in as in the workspace's flag; the caller clears it).  A call needing more scratch
 * (ne_paged_attention_workspace_size() > NE_NOALLOC_SCRATCH_BYTES) returns NE_EWORKSPACE
 * without launching.  It allocates nothing: the scratch address is looked up once per
 * device (hipGetSymbolAddress) on the first call with that device current.  Every call on
 * one GPU shares that GPU's scratch, so calls that overlap on one GPU (concurrent streams)
 * race; calls ordered on one stream do not.
 */
#define NE_NOALLOC_SCRATCH_BYTES (64u << 20)
int ne_paged_verify_attention_noalloc(
    const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k_cache,
    const void* v_cache, const void* k_scale, const void* v_scale, int32_t kv_dtype,
    int32_t scale_dtype, const int32_t* block_tables, int32_t block_table_stride,
    int32_t block_size, const int32_t* ctx_len, const int32_t* q_start, const int32_t* q_len,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t max_q_len, int32_t max_ctx_len, float softmax_scale, void* out,
    int64_t out_token_stride, int64_t out_head_stride, int32_t split_len, uint32_t* error_flag,
    void* stream);

/*
 * A6 with the work plan computed once per step.  ne_paged_attention_plan writes into
 * `workspace` the work item of every work-group and the slot of every 16-key tile,
 * from the same per-step metadata the attention call takes (it replaces the part of
 * batch_builder.py:22-65 / paged_allocator.py:69-79 that turns block tables into
 * context slots, once for all layers).  ne_paged_verify_attention_planned then takes
 * exactly ne_paged_verify_attention's arguments and reads that plan instead of
 * deriving it, which saves one dependent memory round trip per call.  Valid while
 * ctx_len, q_start, q_len, block_tables, num_seqs, max_q_len, max_ctx_len and
 * split_len stay as they were for the plan (a verify step's layers).  Both serve caches
 * with 8 KV heads and at most 32 query rows per KV head (num_q_heads / num_kv_heads *
 * max_q_len <= 32, i.e. up to k = 15 drafts), bf16 or int8 with 2-byte scales, and return
 * NE_EUNSUPPORTED otherwise; the workspace size is ne_paged_attention_workspace_size()'s
 * and its layout does not depend on the cache dtype.
 */
int ne_paged_attention_plan(const int32_t* block_tables, int32_t block_table_stride,
                            int32_t block_size, const int32_t* ctx_len, const int32_t* q_start,
                            const int32_t* q_len, int32_t num_seqs, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t max_q_len, int32_t max_ctx_len,
                            int32_t split_len, void* workspace, size_t workspace_bytes,
                            void* stream);
int ne_paged_verify_attention_planned(
    const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k_cache,
    const void* v_cache, const void* k_scale, const void* v_scale, int32_t kv_dtype,
    int32_t scale_dtype, const int32_t* block_tables, int32_t block_table_stride,
    int32_t block_size, const int32_t* ctx_len, const int32_t* q_start, const int32_t* q_len,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t max_q_len, int32_t max_ctx_len, float softmax_scale, void* out,
    int64_t out_token_stride, int64_t out_head_stride, int32_t split_len, void* workspace,
    size_t workspace_bytes, void* stream);

/* Measurement entry point, no counterpart in the reference: the K/V (and scale) reads of
 * ne_paged_verify_attention_planned alone.  It follows the plan that
 * ne_paged_attention_plan wrote into `workspace` for the same metadata, gives every wave
 * the same tiles and streams them through the same LDS ring with the same copies, and
 * computes and stores nothing.  Its time is what the planned call's access pattern costs
 * the memory system: the ceiling that call is measured against (bench.py).  Same shapes
 * as the planned call; NE_EUNSUPPORTED otherwise. */
int ne_paged_kv_stream_planned(const void* k_cache, const void* v_cache, const void* k_scale,
                               const void* v_scale, int32_t kv_dtype, int32_t scale_dtype,
                               int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t max_q_len, int32_t max_ctx_len, int32_t split_len,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Measurement entry points, no counterpart in the reference: the same K/V bytes read in
 * whole-slot runs.  ne_paged_kv_runs_plan takes the sequences' 16-key tiles in order and
 * cuts them into the workspace's plan_grid runs of near-equal length, across sequence
 * boundaries.  It writes them where ne_paged_attention_plan writes its work items, so a
 * planned call afterwards needs a fresh ne_paged_attention_plan.  ne_paged_kv_stream_runs
 * then reads all 8 KV heads of every tile of run w in work-group w, through the planned
 * call's LDS ring, copies and waits, and computes and stores nothing.  Its time is the
 * stream of a balanced whole-slot split.  ne_paged_kv_stream_planned gives the stream of
 * the planned call's own split, for comparison.  Same shapes, workspace and block-table
 * contract as ne_paged_attention_plan. */
int ne_paged_kv_runs_plan(const int32_t* block_tables, int32_t block_table_stride, int32_t block_size,
                          const int32_t* ctx_len, int32_t num_seqs, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t max_q_len, int32_t max_ctx_len, void* workspace,
                          size_t workspace_bytes, void* stream);
int ne_paged_kv_stream_runs(const void* k_cache, const void* v_cache, const void* k_scale,
                            const void* v_scale, int32_t kv_dtype, int32_t scale_dtype, int32_t num_seqs,
                            int32_t num_q_heads, int32_t num_kv_heads, int32_t max_q_len,
                            int32_t max_ctx_len, void* workspace, size_t workspace_bytes, void* stream);

/*
 * A8 - W8A16 projection: y[m, n] = bf16(sum_k x[m, k] * w[n, k] * scale[n])
 * with int8 weights dequantised in registers onto bf16 MFMA (replaces
 * Int8Linear.forward, ne/models/int8_quantization.py:55-57, which materialises
 * bf16(int8 * scale) and calls F.linear).
 *   x [m, k] bf16 (row stride ldx), w [n, k] int8, scale [n] bf16/fp16/fp32,
 *   y [m, n_out] bf16 (row stride ldy); n_out = n, or n/2 for NE_EPILOGUE_SWIGLU
 *   where weight rows come in groups of 32 (16 gate rows then 16 up rows) and
 *   y[:, 16*i + j] = bf16(silu(gate) * up) for the pair in group i, row j.
 * Requires k % 128 == 0 and n % 64 == 0.
 */
int ne_w8a16_gemm(const void* x, int64_t ldx, const int8_t* w, const void* scale,
                  int32_t scale_dtype, int32_t m, int32_t n, int32_t k, void* y, int64_t ldy,
                  int32_t epilogue, void* stream);

/*
 * A8 (split over K) - the same product as ne_w8a16_gemm's store epilogue, with K
 * cut into `splits` equal parts computed by separate work-groups:
 * partials[s, m, n] = scale[n] * sum_{k in part s} x[m, k] w[n, k], fp32,
 * contiguous [splits, m, n].  For the short, narrow o_proj / down_proj shapes
 * (N = hidden), which alone give too few output tiles to fill the GPU;
 * ne_splitk_add_rmsnorm consumes the partials.  Requires k % (128 * splits) == 0,
 * n % 64 == 0, 1 <= splits <= 64.  A work-group computes 48 token rows x 64 weight
 * rows of one part; for 320 rows of the 0.6B model's o / down, 2 splits (224
 * work-groups) with the norm after them are the fastest measured.
 */
int ne_w8a16_gemm_splitk(const void* x, int64_t ldx, const int8_t* w, const void* scale,
                         int32_t scale_dtype, int32_t m, int32_t n, int32_t k, int32_t splits,
                         float* partials, void* stream);

/*
 * A8b - bf16 GEMM for the tied LM head: logits[m, n] = bf16(sum_k x[m,k] w[n,k])
 * (replaces compute_logits, ne/models/qwen3.py:197-203).  Either output may be
 * null.  When argmax_partials is given, it receives per row ne_lm_head_num_tiles(n)
 * keys, each the largest bf16-rounded logit of a disjoint set of columns with its first
 * index, packed for an ordered max (the row's argmax is the largest key as an unsigned
 * 64-bit integer; its low 32 bits hold 0xFFFFFFFF - column; 0 marks an empty set), for
 * ne_accept to finish.  The sets are each work-group's column range split into the two
 * 128-column halves of its 256-column blocks: ne_lm_head_num_tiles(n) = 2 * min(n / 64,
 * 256); n <= 2^24.  At most 80 rows run a kernel of their own (each wave 32 columns
 * against all rows) that gives the same logits and keys, bit for bit.
 */
int32_t ne_lm_head_num_tiles(int32_t n);
int ne_lm_head(const void* x, int64_t ldx, const void* w, int32_t m, int32_t n, int32_t k,
               void* logits, int64_t ld_logits, uint64_t* argmax_partials, void* stream);

/*
 * RMSNorm pieces of the Qwen3 layer (ne/models/qwen3.py:31-44, 147-150, 178):
 * out = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * weight).
 * ne_rmsnorm:      h = x
 * ne_add_rmsnorm:  h = bf16(residual + delta); residual is updated in place
 * ne_embed_rmsnorm: h = embed[token]; residual = h (ne/models/qwen3.py:167)
 * All tensors bf16, rows of `hidden` elements, contiguous.
 */
int ne_rmsnorm(const void* x, const void* weight, void* out, int32_t rows, int32_t hidden,
               float eps, void* stream);
int ne_add_rmsnorm(void* residual, const void* delta, const void* weight, void* out, int32_t rows,
                   int32_t hidden, float eps, void* stream);
/* ne_add_rmsnorm with delta = bf16(sum_s partials[s, row, :]) taken from the fp32
 * output of ne_w8a16_gemm_splitk ([splits, rows, hidden], 16-byte aligned, splits
 * one of 1, 2, 3, 4, 6, 8); the
 * projection output is rounded to bf16 before the residual add, as in the
 * reference's bf16 o_proj / down_proj followed by the residual add
 * (ne/models/qwen3.py:145-149). */
int ne_splitk_add_rmsnorm(void* residual, const float* partials, int32_t splits, const void* weight,
                          void* out, int32_t rows, int32_t hidden, float eps, void* stream);
int ne_embed_rmsnorm(const int32_t* tokens, const void* embed, const void* weight, void* residual,
                     void* out, int32_t rows, int32_t hidden, float eps, void* stream);

/*
 * Fused QK-norm + RoPE + KV write for one layer (ne/models/qwen3.py:100-104,
 * 47-68, ne/models/attention_context.py:77-94).  qkv [rows, (Hq+2*Hkv)*128] bf16
 * holds q | k | v per row.  q_out [rows, Hq, 128] receives RoPE(q_norm(q)); the
 * key RoPE(k_norm(k)) and value v are written (quantised for an int8 cache) at
 * slot_mapping[row].  rope_cos_sin [rope_positions][2][64] bf16 holds, per
 * position p, bf16(cos(p * inv_freq[i])) then bf16(sin(...)), i < 64, with the
 * fp32 angles of build_rotary_tables (qwen3.py:47-57); dims i and i + 64 share
 * them.  Positions are clamped to the table.
 */
int ne_qk_norm_rope_kv_write(const void* qkv, int32_t rows, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, const void* q_norm_weight,
                             const void* k_norm_weight, float eps, const int32_t* positions,
                             const void* rope_cos_sin, int32_t rope_positions,
                             const int32_t* slot_mapping, void* k_cache, void* v_cache,
                             void* k_scale, void* v_scale, int32_t kv_dtype, int32_t scale_dtype,
                             void* q_out, void* stream);

/*
 * A8 + A7 fused for the QKV projection: the W8A16 product of ne_w8a16_gemm (store
 * epilogue) over the concatenated q | k | v weight ([(Hq+2*Hkv)*128, k] int8,
 * per-row scales), each 128-wide head of every row then taken exactly as
 * ne_qk_norm_rope_kv_write takes it (the same bits), without writing the qkv
 * product to memory.  Replaces Int8Linear.forward of q_proj/k_proj/v_proj
 * (ne/models/int8_quantization.py:55-57, ne/models/qwen3.py:95-98) followed by
 * qwen3.py:100-104 and write_to_cache (ne/models/attention_context.py:42-54).
 * kv_dtype NE_DTYPE_INT8 (scales bf16 or fp16) or NE_DTYPE_BF16; k % 128 == 0;
 * x and w 16-byte aligned.
 */
int ne_w8a16_qkv_norm_rope_kv(const void* x, int64_t ldx, const int8_t* w, const void* scale,
                              int32_t scale_dtype, int32_t m, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t k, const void* q_norm_weight,
                              const void* k_norm_weight, float eps, const int32_t* positions,
                              const void* rope_cos_sin, int32_t rope_positions,
                              const int32_t* slot_mapping, int32_t kv_dtype, void* k_cache,
                              void* v_cache, void* k_scale, void* v_scale, int32_t kv_scale_dtype,
                              void* q_out, void* stream);

/*
 * A9/A10 - fused acceptance (replaces verify_proposal and the sampling helpers,
 * ne/engine/speculative/verifier.py:21-60, ne/engine/sampling.py:21-42, and the
 * rollback of ne/engine/speculative/speculative_generator.py:78-83).
 * Sequence b has num_drafts[b] guesses drafts[b, :] and target rows
 * row_start[b] .. row_start[b]+num_drafts[b] (one more than its guesses).
 * temperature[b] (device fp32; null: every sequence greedy) selects per sequence:
 * Greedy (temperature 0): target token of a row = argmax of its bf16 logits, first
 * index on ties, from `logits` or, when logits is null, from the ne_lm_head
 * partials.  Keep guesses while guess == target; then append the target of the
 * first mismatching row (or the bonus row).
 * Sampled (temperature > 0): p' = softmax(fp32(logit) / T), cut to top_p[b]
 * (device fp32; null: 1) and renormalised (sampling.py:21-38), under the fixed-order
 * contract documented in accept.hip; guess i is kept iff p'_i >= 1 or (p'_i > 0 and
 * u_i < p'_i); a rejection resamples from p' with the guess removed (p' itself if
 * that is empty) and the bonus samples p' of the last row, both by inverse CDF with
 * u_draw.  Uniforms u_i, u_draw come from Philox4x32-10 keyed by seeds[b] at
 * counter (steps[b], j/4), word j%4, j = i (guesses) and 63.  any_sampled must be
 * non-zero when some temperature is positive (logits, seeds and steps are then
 * required).
 * draft_rows (sampled sequences; guesses drawn by a draft model): the draft's
 * distribution for guess i of sequence b is row draft_row_start[b] + i (stride
 * ld_draft) -- bf16 logits (draft_dtype NE_DTYPE_BF16; q = the same temperature /
 * top-p softmax) or fp32 probabilities used as given (NE_DTYPE_FP32); guess i is
 * kept iff a = min(p'/max(q,1e-12), 1) >= 1 or (a > 0 and u_i < a), and a rejection
 * draws from max(p' - q, 0) (p' when that is empty), verifier.py:36-56.  Null: the
 * guesses are deterministic (one-hot q), as above.
 * Outputs: out_tokens[b, 0..num_out[b]-1] (kept guesses + 1 target token),
 * the rest of the row [b, 0..max_drafts] set to -1; num_out[b] = kept + 1.  When
 * history is given, the kept tokens and the target token are appended at
 * history[b, history_len[b]..] (within the row's history_stride tokens) and
 * history_len[b] and num_cached[b] (set to history_len_before + kept) are updated; a
 * sequence whose history_len is 0 is inactive (num_out 0, nothing written).
 */
int ne_accept(const void* logits, int64_t ld_logits, const uint64_t* argmax_partials,
              int32_t num_tiles, int32_t vocab, const int32_t* drafts, int32_t max_drafts,
              const int32_t* num_drafts, const int32_t* row_start, int32_t num_seqs,
              const float* temperature, const float* top_p, int32_t any_sampled,
              const uint64_t* seeds, const uint64_t* steps, int32_t* out_tokens, int32_t* num_out,
              int32_t* history, int64_t history_stride, int32_t* history_len, int32_t* num_cached,
              const void* draft_rows, int32_t draft_dtype, int64_t ld_draft,
              const int32_t* draft_row_start, void* stream);

/*
 * Device-side packing of a batched verify step (replaces build_step_inputs,
 * ne/engine/generation/batch_builder.py:22-65, and the slot arithmetic of
 * ne/engine/memory/paged_allocator.py:69-79 for the verify step).  Sequence b
 * owns rows b*R .. b*R+R-1, R = max_drafts + 1: row 0 is the last accepted token
 * history[b, L-1] at position L-1 (L = history_len[b]), row i <= num_drafts[b]
 * is guess i-1 at position L-1+i; the remaining rows are padding (token 0,
 * position 0, scratch_slot).  Writes q_start = b*R, q_len = num_drafts+1 and
 * ctx_len = L + num_drafts; history_len 0 marks an inactive slot (q_len 0).
 */
int ne_prepare_verify_step(const int32_t* history, int64_t history_stride,
                           const int32_t* history_len, const int32_t* drafts, int32_t max_drafts,
                           const int32_t* num_drafts, const int32_t* block_tables,
                           int32_t block_table_stride, int32_t block_size, int32_t scratch_slot,
                           int32_t num_seqs, int32_t* tokens, int32_t* positions,
                           int32_t* slot_mapping, int32_t* q_start, int32_t* q_len,
                           int32_t* ctx_len, void* stream);

/*
 * Counters of the next verify step, advanced on the device after ne_accept so that
 * the next step's n-gram proposal can run without a host round trip (replaces the
 * per-step num_guesses of ne/engine/speculative/speculative_generator.py:71-72 and
 * the generator's step counter).  For every sequence b with history_len[b] > 0:
 * num_generated[b] += num_out[b]; steps[b] += 1;
 * num_guesses[b] = max(0, min(k, max_new_tokens[b] - num_generated[b] - 1)).
 * Sequences with history_len 0 are inactive: num_guesses[b] = 0, nothing else written.
 */
int ne_advance_step_counts(const int32_t* history_len, const int32_t* num_out,
                           const int32_t* max_new_tokens, int32_t* num_generated, uint64_t* steps,
                           int32_t* num_guesses, int32_t k, int32_t num_seqs, void* stream);

/*
 * ne_advance_step_counts followed by ne_ngram_propose in one launch (the tail of a
 * verify step: speculative_generator.py:71-72, then NgramProposer.propose of
 * ne/engine/speculative/proposers.py:39-57 for the next step).  The work-group of
 * sequence b advances b's counters exactly as ne_advance_step_counts does, writes
 * num_guesses[b], and proposes up to min(num_guesses[b], max_drafts) guesses from b's
 * history as ne_ngram_propose does with num_tokens = num_guesses.
 */
int ne_advance_and_propose(const int32_t* history, int64_t history_stride, const int32_t* history_len,
                           const int32_t* num_out, const int32_t* max_new_tokens, int32_t* num_generated,
                           uint64_t* steps, int32_t* num_guesses, int32_t k, int32_t num_seqs,
                           int32_t max_ngram, int32_t min_ngram, int32_t max_drafts, int32_t* drafts,
                           int32_t* num_drafts, void* stream);

/* Plain device copy of `bytes` bytes (16-byte aligned); used to calibrate the
 * hardware byte counters against a kernel of known traffic. */
int ne_copy_bytes(const void* src, void* dst, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOENGINE_HIP_H */
