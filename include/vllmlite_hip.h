/*
 * C ABI of the MI355X (gfx950) ragged paged-attention step.
 *
 * Conventions shared by every entry point:
 *   - pointers are device pointers unless the parameter name ends in _host;
 *   - `stream` is a hipStream_t (NULL = the null stream); work is enqueued
 *     asynchronously and nothing synchronises;
 *   - no entry point allocates device memory; scratch space is passed in as
 *     `workspace` / `workspace_bytes`;
 *   - the return value is 0 (VL_OK), a negative VL_E* argument error, or a
 *     positive hipError_t; vl_last_error() returns the message of the last
 *     failure on the calling thread. Nothing throws across this boundary.
 *   - dtype is VL_DTYPE_F32 (float) or VL_DTYPE_BF16 (raw bfloat16 bits);
 *     the paged-attention calls also take VL_DTYPE_F32_BF16KV and
 *     VL_DTYPE_F32_FP8KV: fp32 query and output over bf16 or FP8 E4M3
 *     caches (a narrow KV cache under an fp32 model). FP8 E4M3 is the OCP
 *     format (4 exponent bits, bias 7, 3 mantissa bits, no infinities, 0x7F
 *     / 0xFF NaN, largest finite 448); writers round to nearest even and
 *     saturate finite values beyond 448 to +-448.
 *
 * Cache layout (kv_layout): VL_KV_TOKEN_MAJOR is the reference's
 * (vllmlite/runner.py:41-44), one tensor per layer and per K/V of shape
 * [num_slots, num_kv_heads, head_dim], where slot = block_id * block_size +
 * offset (vllmlite/block.py:154-156). VL_KV_HEAD_MAJOR stores the same
 * blocks as [num_blocks, num_kv_heads, block_size, head_dim]: one KV head's
 * rows of a block are contiguous (block_size must be a power of two). Slots,
 * block tables and block copies are the same in both; only the order of the
 * rows inside a block differs.
 */
#ifndef VLLMLITE_HIP_H
#define VLLMLITE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VL_OK 0
#define VL_EINVAL (-1)
#define VL_DTYPE_F32 0
#define VL_DTYPE_BF16 1
#define VL_DTYPE_F32_BF16KV 2
#define VL_DTYPE_FP8_E4M3 3   /* cache elements: OCP FP8 E4M3 (e4m3fn) bytes */
#define VL_DTYPE_F32_FP8KV 4  /* attention: fp32 query and output over FP8 E4M3 caches */
#define VL_KV_TOKEN_MAJOR 0 /* caches [num_slots, num_kv_heads, head_dim] */
#define VL_KV_HEAD_MAJOR 1  /* caches [num_blocks, num_kv_heads, block_size, head_dim] */
#define VL_LINEAR_STORE 0      /* vl_linear_rows: out = f(x) @ W */
#define VL_LINEAR_ACCUMULATE 1 /* out += f(x) @ W (the residual add) */
#define VL_LINEAR_SWIGLU 2     /* out = silu(f(x) @ W[:, :n]) * (f(x) @ W[:, n:2n]) */
#define VL_LINEAR_TILES16 16   /* flag ORed into the mode: W in 16-column tiles */
#define VL_WEIGHT_ROWS 0       /* a projection weight [k, n] row-major at a row stride */
#define VL_WEIGHT_TILES16 1    /* ... as 16-column tiles [ceil(n/16), k, 16], zero past n;
                                  inside a tile, element (k, m) with k = 16g + 4j + s
                                  at flat position 256g + 4(16j + m) + s */

/* Message of the last failed call on this thread ("" if none). */
const char* vl_last_error(void);

/* ABI revision of this library; bumped when a signature changes. */
int vl_abi_version(void);

/*
 * K1 reshape-and-cache. Replaces write_kv (vllmlite/attention.py:47-49) as
 * called per sequence per layer at vllmlite/model.py:109:
 *   key_cache[slot_mapping[t]] = key[t]; value_cache[slot_mapping[t]] = value[t]
 * for t < num_tokens. key/value rows are [num_kv_heads, head_dim] contiguous,
 * `key_stride`/`value_stride` elements apart. A negative slot skips the token.
 * The caches are kv_layout (block_size is read only for VL_KV_HEAD_MAJOR).
 * dtype VL_DTYPE_F32, VL_DTYPE_BF16 or VL_DTYPE_FP8_E4M3 (inputs and caches
 * alike). Bit-exact copy.
 */
int vl_reshape_and_cache(const void* key, const void* value, int64_t key_stride,
                         int64_t value_stride, void* key_cache, void* value_cache,
                         const int32_t* slot_mapping, int64_t num_tokens, int num_kv_heads,
                         int head_dim, int dtype, int kv_layout, int block_size, void* stream);

/*
 * K3 copy-on-write block copy. Replaces NumpyRunner._do_cow
 * (vllmlite/runner.py:54-60): for each pair (src, dst) of `block_pairs`
 * [num_pairs, 2] and each layer l < num_layers, copies block_elems elements
 * from base + l*layer_stride + src*block_elems to ... + dst*block_elems, for
 * the K and the V cache. Pairs are processed in parallel, which equals the
 * reference's in-order loop because no dst is another pair's src and dsts are
 * distinct (fresh blocks, vllmlite/block_manager.py:77-85); the caller must
 * guarantee that. dtype VL_DTYPE_F32, VL_DTYPE_BF16 or VL_DTYPE_FP8_E4M3.
 * Bit-exact copy.
 */
int vl_copy_blocks(void* key_cache, void* value_cache, const int32_t* block_pairs, int num_pairs,
                   int num_layers, int64_t layer_stride, int64_t block_elems, int dtype,
                   void* stream);

/*
 * Workspace bytes vl_paged_attention works best with for this batch shape.
 * Any size >= vl_paged_attention_min_workspace() is correct: with less room
 * the kernel splits long contexts into fewer partitions.
 */
size_t vl_paged_attention_workspace_size(int num_seqs, int num_tokens, int num_heads,
                                         int head_dim, int max_context_len);
size_t vl_paged_attention_min_workspace(int num_seqs);

/*
 * K2 ragged paged attention, decode + chunked prefill + speculative verify in
 * one call. Replaces paged_attention (vllmlite/attention.py:59-98) called per
 * sequence at vllmlite/model.py:107-112. Sequence i owns query tokens
 * [query_start_loc[i], query_start_loc[i+1]) of `query` [num_tokens, num_heads,
 * head_dim] (rows `query_stride` elements apart) and seq_lens[i] cached tokens
 * (this step's K/V already written) reached through block_tables[i,
 * 0..ceil(seq_lens[i]/block_size)). Query j of a sequence with q_len tokens
 * sits at position seq_lens[i] - q_len + j and attends keys 0..position
 * (causal; a single query sees the whole context). Head h reads KV head
 * h / (num_heads / num_kv_heads). The caches are kv_layout. out [num_tokens,
 * num_heads, head_dim], contiguous, dtype of the query. Accumulation is fp32.
 * Launch hints, each 0 when unknown: max_query_len and min_query_len bound
 * the query count of the sequences with at least one query, max_context_len
 * bounds seq_lens. With max_query_len 1 and max_context_len <= 2048, head_dim
 * 16, 32, 48 or 64, 1, 2, 4 or 8 query heads per KV head and a power-of-two
 * block size, one short-decode launch runs the call and reads no plan (the
 * _plan call may be skipped; vl_paged_attention skips it). For bf16,
 * head_dim 128, 4 query heads per KV head and 16-token blocks: max 1 launches
 * only the decode kernel, min 1 with max > 1 (decodes and multi-query
 * sequences) only the one-launch step kernel, min > 1 only the multi-query
 * kernels; with a bound unknown the kernels decide on the device. Bounds that
 * do not hold leave some sequences' outputs unwritten (nothing is read or
 * written out of bounds).
 */
int vl_paged_attention(void* out, const void* query, int64_t query_stride, const void* key_cache,
                       const void* value_cache, const int32_t* block_tables,
                       int block_table_stride, const int32_t* seq_lens,
                       const int32_t* query_start_loc, int num_seqs, int num_tokens,
                       int num_heads, int num_kv_heads, int head_dim, int block_size,
                       float scale, int dtype, int kv_layout, int max_query_len,
                       int min_query_len, int max_context_len, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * The two halves of vl_paged_attention, for callers that run several
 * attention calls over the same batch (one per layer): _plan reads only
 * seq_lens / query_start_loc and writes the work decomposition into the
 * workspace; _run performs the attention using the plan currently in that
 * workspace, which must come from a _plan call with the same lengths, head
 * counts, head_dim, block_size, dtype and workspace size (stream-ordered before
 * it; the plan does not depend on kv_layout). vl_paged_attention is _plan
 * followed by _run. A run also uses the workspace as scratch (split partials,
 * work and arrival counters, which it leaves at zero for the next run of the
 * same plan): runs on one workspace must not overlap (one stream, or ordered
 * by events).
 */
int vl_paged_attention_plan(const int32_t* seq_lens, const int32_t* query_start_loc,
                            int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
                            int head_dim, int block_size, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream);
int vl_paged_attention_run(void* out, const void* query, int64_t query_stride,
                           const void* key_cache, const void* value_cache,
                           const int32_t* block_tables, int block_table_stride,
                           const int32_t* seq_lens, const int32_t* query_start_loc, int num_seqs,
                           int num_tokens, int num_heads, int num_kv_heads, int head_dim,
                           int block_size, float scale, int dtype, int kv_layout,
                           int max_query_len, int min_query_len, int max_context_len,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * 1 if a _run call with these shapes and launch hints reads the plan, 0 if it
 * takes the short-decode kernel, which reads none (its _plan call may then be
 * skipped). Part of this library's plan/run split; the reference has no plan.
 */
int vl_paged_attention_reads_plan(int num_heads, int num_kv_heads, int head_dim, int block_size,
                                  int max_query_len, int max_context_len);

/*
 * vl_paged_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * Its workspace is a static device array of VL_NOALLOC_SCRATCH_BYTES bytes,
 * one per GPU, held until the process ends; the call allocates nothing and
 * calls no allocating routine. Batches whose plan alone needs more than that
 * (vl_paged_attention_min_workspace(num_seqs) > VL_NOALLOC_SCRATCH_BYTES) are
 * rejected with VL_EINVAL; smaller ones run exactly as vl_paged_attention
 * with a workspace of that size. Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, two threads) race and must be
 * ordered by the caller. Each call rewrites all plan state before reading it.
 */
#define VL_NOALLOC_SCRATCH_BYTES (32u << 20)
int vl_paged_attention_noalloc(void* out, const void* query, int64_t query_stride,
                               const void* key_cache, const void* value_cache,
                               const int32_t* block_tables, int block_table_stride,
                               const int32_t* seq_lens, const int32_t* query_start_loc,
                               int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
                               int head_dim, int block_size, float scale, int dtype,
                               int kv_layout, int max_query_len, int min_query_len,
                               int max_context_len, void* stream);

/*
 * K4a RMSNorm, optionally fused with the residual add that precedes it
 * (vllmlite/model.py:17-19 used at 96, 116, 119):
 *   if residual != NULL: residual[r] += x[r] (x = residual afterwards)
 *   out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * weight
 * rows of `dim` floats, fp32 only.
 */
int vl_rms_norm(float* out, float* residual, const float* x, const float* weight, int64_t rows,
                int dim, float eps, void* stream);

/*
 * SwiGLU gate of the TinyLlama MLP (vllmlite/model.py:22-23, 117): for a
 * fused projection gate_up [rows, 2*d_ff] = [h@w_gate | h@w_up],
 * out[r, j] = silu(gate) * up with silu(x) = x / (1 + exp(-x)). fp32 only.
 */
int vl_silu_mul(float* out, const float* gate_up, int64_t rows, int d_ff, void* stream);

/*
 * K4b RoPE fused with the K/V scatter. For a fused projection row
 * qkv[t] = [q (num_heads*head_dim) | k (num_kv_heads*head_dim) | v (...)]
 * (`qkv_stride` elements apart), rotates interleaved (even, odd) pairs of q
 * and k by cos/sin[positions[t]] (tables [max_pos, head_dim/2], fp32;
 * vllmlite/attention.py:21-37), writes rotated q to q_out [num_tokens,
 * num_heads, head_dim] and rotated k / plain v to the caches at
 * slot_mapping[t] (vllmlite/attention.py:47-49). fp32 arithmetic; the caches
 * hold cache_dtype elements (VL_DTYPE_F32; VL_DTYPE_BF16 or
 * VL_DTYPE_FP8_E4M3: each value rounded to nearest even when stored, FP8
 * saturating at +-448) in kv_layout (block_size is read only for
 * VL_KV_HEAD_MAJOR).
 */
int vl_rope_and_cache(const float* qkv, int64_t qkv_stride, float* q_out, void* key_cache,
                      void* value_cache, const int32_t* positions, const int32_t* slot_mapping,
                      const float* cos_table, const float* sin_table, int64_t num_tokens,
                      int num_heads, int num_kv_heads, int head_dim, int cache_dtype,
                      int kv_layout, int block_size, void* stream);

/*
 * K6 fp32 projections of the TinyLlama forward for at most 16 token rows
 * (the decode steps), with their neighbours fused: f(x) = x, or when
 * norm_weight != NULL the RMSNorm of each row of x times norm_weight (as
 * vl_rms_norm computes it), then by mode
 *   VL_LINEAR_STORE       out = f(x) @ W           (q/k/v: model.py:96-101;
 *                                                  lm_head: model.py:119-120)
 *   VL_LINEAR_ACCUMULATE  out += f(x) @ W          (the residual adds,
 *                                                  model.py:114, 117)
 *   VL_LINEAR_SWIGLU      out = silu(f(x) @ W[:, :n]) * (f(x) @ W[:, n:2n])
 *                                                  (model.py:116-117, with
 *                                                  W = [w_gate | w_up])
 * x [*, k] (16-byte aligned, row stride a multiple of 4); row r of the
 * input is x[row_index[r]] when row_index != NULL (the gather of the logits
 * rows, runner.py:90), else x[r]. W [k, n] (or [k, 2n]) row-major with row
 * stride weight_stride, or, with VL_LINEAR_TILES16 ORed into mode, as
 * 16-column tiles [ceil(n/16), k, 16] (zero past column n; SwiGLU: the gate
 * tiles, then the up tiles; weight_stride unused; 16-byte aligned; inside a
 * tile element (k, m), k = 16g + 4j + s, at flat position 256g + 4(16j + m) +
 * s, so each lane's operands of 4 MFMA steps are one 16-byte load, as are
 * the x elements they meet; norm_weight, when given, 16-byte aligned). out [rows, n]; out must not overlap x. rows <= 16 * 65535
 * (a workgroup per 16 columns and 16 rows, or 2 or 4 row tiles in turn on large
 * grids; built for the <= 16 rows of a decode step, where one row tile does
 * it), k a multiple of 16, k <= 1024.
 * fp32 throughout.
 */
int vl_linear_rows(float* out, int64_t out_stride, const float* x, int64_t x_stride,
                   const int32_t* row_index, const float* weight, int64_t weight_stride,
                   const float* norm_weight, float eps, int rows, int k, int n, int mode,
                   void* stream);

/*
 * vl_linear_rows in VL_LINEAR_STORE mode over tiled weights (the lm_head of
 * vllmlite/model.py:119-120 on the gathered rows, runner.py:90) that also
 * writes each row's argmax over its n logits to ids[rows], and to host_ids
 * when it is not NULL (pinned host memory the host polls): greedy sampling,
 * sampling.py:56-57, with numpy's rule (the lowest index among equal
 * maxima, -0 equal to +0, the first NaN beating every number), as
 * vl_argmax_rows computes it, in the same launch. scratch: 8 (rows + 1)
 * bytes, 8-byte aligned, zero before the first call; every call leaves it
 * zero again (calls that overlap on one scratch race). ids are written by
 * the launch's last workgroup after every logit is stored.
 */
int vl_linear_rows_argmax(float* out, int64_t out_stride, const float* x, int64_t x_stride,
                          const int32_t* row_index, const float* weight, const float* norm_weight,
                          float eps, int rows, int k, int n, int32_t* ids, int32_t* host_ids,
                          void* scratch, int64_t scratch_bytes, void* stream);

/*
 * vl_linear_rows in VL_LINEAR_SWIGLU mode over tiled weights, with the input
 * rows x[r] + x_parts[r, 0] + ... + x_parts[r, num_parts - 1] (x_parts
 * [rows, num_parts, k] fp32, summed in that order; num_parts 1, 2, 4 or 8;
 * k <= 512): the residual add of vllmlite/model.py:114 (x + attn @ wo, wo's
 * product arriving as one partial row per KV head from
 * vl_decode_attention_wo) fused into the RMSNorm + gate|up + SwiGLU of
 * model.py:116-117. When x_out != NULL (not x) the summed rows are written
 * there too [rows, k], the residual the down projection adds to.
 */
int vl_linear_rows_parts(float* out, int64_t out_stride, const float* x, int64_t x_stride,
                         const float* x_parts, int num_parts, float* x_out, const float* weight,
                         const float* norm_weight, float eps, int rows, int k, int n,
                         void* stream);

/*
 * K6b the QKV projection of a step's rows fused with RoPE and the K/V
 * scatter (vllmlite/model.py:96-103, 109; vllmlite/attention.py:21-37,
 * 47-49): qkv = f(x) @ weight (weight [k, (num_heads + 2 num_kv_heads) *
 * head_dim], f as in vl_linear_rows), then exactly what vl_rope_and_cache
 * does with that row: rotated q to q_out [rows, num_heads * head_dim],
 * rotated k and plain v to the caches at slot_mapping[r] (skipped when < 0).
 * Input rows are x[row_index[r]] when row_index != NULL (the embedding
 * gather tok_emb[token_ids], model.py:93); an index -(1 + i) < 0 stands for
 * prev_ids[i] (0 when i >= num_prev), the id the previous step chose for its
 * row i, as vl_resolve_tokens would replace it (prev_ids may be NULL when
 * num_prev is 0). When x_out != NULL the rows
 * read (before the norm) are also written to x_out [rows, k] (the residual
 * stream). weight_layout: VL_WEIGHT_ROWS (row stride weight_stride) or
 * VL_WEIGHT_TILES16 (as for vl_linear_rows). rows <= 16 * 65535, k a multiple
 * of 16, k <= 1024, head_dim even. fp32; the caches hold cache_dtype elements in
 * kv_layout as for vl_rope_and_cache. When record_words > 0 the launch also
 * copies record_src[0 .. record_words) to record_dst (ABI 13; no reference
 * counterpart): a step's int32 record from pinned host memory to the device
 * in the step's first launch, instead of a copy launch before it.
 * row_index, positions and slot_mapping may then point into record_src (they
 * are read from there); record_dst must not overlap anything the launch
 * reads, and holds the copy once the launch has ended.
 */
int vl_qkv_rope_cache(float* q_out, void* key_cache, void* value_cache, const float* x,
                      int64_t x_stride, const int32_t* row_index, const int32_t* prev_ids,
                      int64_t num_prev, float* x_out,
                      const float* weight, int64_t weight_stride, int weight_layout,
                      const float* norm_weight, float eps, const int32_t* positions,
                      const int32_t* slot_mapping, const float* cos_table, const float* sin_table,
                      int rows, int k, int num_heads, int num_kv_heads, int head_dim,
                      int cache_dtype, int kv_layout, int block_size, const int32_t* record_src,
                      int32_t* record_dst, int64_t record_words, void* stream);

/*
 * K2 for a decode batch (every sequence one query; the short-decode kernel's
 * shapes: fp32 queries over fp32 / bf16 / FP8 E4M3 caches, dtype
 * VL_DTYPE_F32 / _F32_BF16KV / _F32_FP8KV, head_dim 16 / 32 / 48 / 64, 1 / 2 /
 * 4 / 8 query heads per KV head, power-of-two blocks, 0 < max_context_len <=
 * 2048) fused with the output projection (vllmlite/attention.py:59-98 then
 * model.py:114's attn @ wo): instead of the attention rows, parts[s, g, :] =
 * (sequence s's outputs of the query heads of KV head g, as one row of
 * heads-per-group x head_dim) @ wo[those rows, 0 .. d_model), wo row-major
 * [num_heads * head_dim, d_model], d_model <= 512. Summed over g (in order)
 * and added to the residual, they are model.py:114's x + attn @ wo
 * (vl_linear_rows_parts does that in the next projection's prologue).
 * Arguments otherwise as vl_paged_attention_run.
 */
int vl_decode_attention_wo(float* parts, const float* query, int64_t query_stride,
                           const void* key_cache, const void* value_cache,
                           const int32_t* block_tables, int block_table_stride,
                           const int32_t* seq_lens, const int32_t* query_start_loc, int num_seqs,
                           int num_heads, int num_kv_heads, int head_dim, int block_size,
                           float scale, int dtype, int kv_layout, int max_context_len,
                           const float* wo, int d_model, void* stream);

/*
 * A copy of n int32 words by one kernel (no counterpart in the reference,
 * which has no device): src may be pinned host memory (hipHostMalloc), read
 * by the kernel over the bus. A step graph's host-to-device copy of its
 * staging record, as a memcpy node, costs ~12 us more per step than this
 * kernel node.
 */
int vl_copy_words(int32_t* dst, const int32_t* src, int64_t n, void* stream);

/*
 * The device side of a step issued before the previous step's tokens reached
 * the host (no reference counterpart: the reference engine waits for every
 * step, vllmlite/engine.py:99-181): token_ids[i] < 0 stands for
 * prev_ids[-token_ids[i] - 1], the id the previous step chose for that row,
 * and is replaced by it in place (0 if the index is not below num_prev).
 */
int vl_resolve_tokens(int32_t* token_ids, int64_t num_tokens, const int32_t* prev_ids,
                      int64_t num_prev, void* stream);

/*
 * K5 greedy acceptance. Replaces verify (vllmlite/speculative.py:86-100).
 * Sequence i owns logits rows row_start[i] .. row_start[i] + num_drafts[i]
 * (vocab floats each, `row_stride` apart) and drafts[i, 0..num_drafts[i]).
 * picked[r] = argmax(row r), ties to the lowest index (numpy's argmax). Writes
 * out_tokens[i, 0..max_drafts] = picked while it equals the draft, then the
 * first mismatch (or, all matched, the bonus row's pick); unused entries -1;
 * num_accepted[i] = drafts accepted. Integer outputs are exact. One launch
 * (ABI 12: before, a pick and an acceptance launch): scratch holds 8 *
 * num_seqs * (max_drafts + 1) + 4 * num_seqs bytes, 8-byte aligned, zero
 * before the first call; every call leaves it zero again (calls that overlap
 * on one scratch race).
 */
int vl_greedy_verify(const float* logits, int64_t row_stride, int vocab, const int32_t* row_start,
                     const int32_t* num_drafts, const int32_t* drafts, int max_drafts,
                     int32_t* out_tokens, int32_t* num_accepted, int num_seqs, void* scratch,
                     int64_t scratch_bytes, void* stream);

/*
 * Row-wise argmax (ties to the lowest index) of rows x vocab fp32 logits into
 * out[rows], and also into out2 when it is not NULL: a second copy in memory
 * the host reads (pinned host memory), written by the same launch instead of
 * a copy behind it. (ABI 6 added out2.)
 */
int vl_argmax_rows(const float* logits, int64_t row_stride, int64_t rows, int vocab, int32_t* out,
                   int32_t* out2, void* stream);

/*
 * K7 one decode step of the TinyLlama forward in one launch
 * (vllmlite/model.py:80-120 over the batch vllmlite/runner.py:62-100 builds
 * when every scheduled sequence pushes one token, then the greedy argmax of
 * vllmlite/sampling.py:56-57 on each logits row). Row r (r < 16) is sequence
 * r: token token_ids[r] (t < 0 stands for prev_ids[-t - 1], the id the
 * previous step chose for its row -t - 1) at positions[r], its K/V written
 * to slot_mapping[r] (< 0: none) and seq_lens[r] tokens of context through
 * block_tables[r, :] (r >= num_seqs, or seq_lens[r] == 0: a padding row,
 * whose outputs are unspecified). Per layer: RMSNorm, QKV, RoPE, the K/V
 * scatter, paged attention, x += attn @ wo, RMSNorm, SwiGLU, x += act @
 * w_down; then the final RMSNorm and lm_head: logits [16, vocab], and the
 * argmax of every row (numpy's rule) into out_ids[16] and out_ids_host[16]
 * (pinned host memory). out_ids_host[16] is left as the caller set it (0)
 * when the launch was good, else set to 1 (a wait between the step's phases
 * ran out) or 2 (the step's workgroups were not all on one XCD): the
 * results are then invalid. Every result equals what this library's
 * separate kernels compute for the step (vl_qkv_rope_cache,
 * vl_paged_attention, vl_linear_rows, vl_argmax_rows).
 *
 * layer_weights: 6 device addresses (a host array), each the first of
 * n_layers buffers of its kind laid out layer_strides[k] floats apart: the
 * attn_norm [d], the fused QKV weight, wo, ffn_norm [d], the fused gate|up
 * weight and w_down, each weight in the 16-column tile layout of
 * VL_WEIGHT_TILES16 ([ceil(n/16), k, 16]; gate|up: the gate tiles, then the
 * up tiles); lm_head likewise. Caches [n_layers] x layer_stride elements of kv_dtype
 * (VL_DTYPE_F32, _BF16 or _FP8_E4M3, written rounded to nearest even) in
 * kv_layout, a layer under 2 GiB. x, q, attn, act: fp32 [16, d], [16, d],
 * [16, d], [16, d_ff] rows the launch exchanges between its phases; sync:
 * 128 uint32 words, 128-byte aligned, zero before the first launch (every
 * launch leaves them so); launches sharing sync words or row buffers must not
 * overlap. vl_decode_step_supported says which shapes have a kernel (today:
 * head_dim 16 or 48, 2 query heads per KV head, d_model <= 384 a multiple
 * of 64, d_ff <= 1024 a multiple of 16, context <= 2048).
 */
int vl_decode_step_supported(int d_model, int num_heads, int num_kv_heads, int d_ff, int kv_dtype,
                             int max_context);
int vl_decode_step(const void* const* layer_weights, const int64_t* layer_strides, int n_layers,
                   const float* tok_emb,
                   const float* final_norm, const float* lm_head, void* key_cache,
                   void* value_cache, int64_t layer_stride, int kv_dtype, int kv_layout,
                   const int32_t* token_ids, const int32_t* positions,
                   const int32_t* slot_mapping, const int32_t* seq_lens,
                   const int32_t* block_tables, int block_table_stride, int num_seqs,
                   const int32_t* prev_ids, int num_prev, const float* cos_table,
                   const float* sin_table, int d_model, int num_heads, int num_kv_heads,
                   int d_ff, int vocab, int block_size, int max_context, float scale, float eps,
                   float* x, float* q, float* attn, float* act, float* logits, int32_t* out_ids,
                   int32_t* out_ids_host, uint32_t* sync, void* stream);

/*
 * A submission thread for captured step graphs (no counterpart in the
 * reference: its engine steps synchronously, vllmlite/engine.py:99-181; the
 * callers are runners that overlap host work with a step in flight).
 * vl_launcher_create starts a thread that launches graph executables on
 * `stream` (of `device`), in submission order; vl_launcher_submit queues
 * hipGraphLaunch(graph_exec) (skipped when NULL) followed by
 * hipEventRecord(event) (skipped when NULL) and returns at once with a
 * ticket (1, 2, ...); vl_launcher_wait returns once the calls of that ticket
 * and every earlier one have returned, with 0 or the first hipError_t any of
 * them gave (the work itself may still be running on the device: wait on
 * the event for that). vl_launcher_destroy launches what is queued, then
 * stops the thread. The graph executables, events and stream must outlive
 * their submissions.
 */
int vl_launcher_create(int device, void* stream, void** launcher);
int vl_launcher_submit(void* launcher, void* graph_exec, void* event, uint64_t* ticket);
int vl_launcher_wait(void* launcher, uint64_t ticket);
int vl_launcher_destroy(void* launcher);
/*
 * Host side: spins until values[0..n) (pinned host memory a kernel writes,
 * the caller having set it negative) are all >= 0, or timeout_us passes
 * (then VL_EINVAL). A step's token ids arrive this way without an event
 * record behind the step's graph (which costs the device 3-4.5 us).
 */
int vl_host_wait_nonneg(const int32_t* values, int64_t n, int64_t timeout_us);

#ifdef __cplusplus
}
#endif
#endif /* VLLMLITE_HIP_H */
