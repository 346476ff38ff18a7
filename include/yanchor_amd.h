/*
 * yanchor_amd C ABI: MI355X (gfx950) kernels for YANchor's batched recurrent
 * decode / prefill hot path.
 *
 * Conventions for every entry point:
 *   - all tensor arguments are device pointers to caller-owned memory; the
 *     library never allocates or frees device memory;
 *   - tensors are dense row-major in the layout written next to each argument;
 *   - `stream` is a hipStream_t (passed as void* so this header needs no HIP
 *     include); work is enqueued on it and the call returns without a sync;
 *   - the return value is 0 (YH_OK) or a negative error code; yh_last_error()
 *     returns a message for the calling thread's last failure;
 *   - dtype codes are the yh_dtype values below.
 */
#ifndef YANCHOR_AMD_H
#define YANCHOR_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* yh_stream_t;

enum yh_dtype { YH_F32 = 0, YH_BF16 = 1, YH_F16 = 2, YH_I32 = 3, YH_I64 = 4, YH_U8 = 5 };

enum yh_status { YH_OK = 0, YH_ERR_INVALID = -1, YH_ERR_HIP = -2, YH_ERR_UNSUPPORTED = -3 };

/* Message describing the calling thread's most recent error ("" if none). */
const char* yh_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int yh_abi_version(void);

/*
 * Gated delta rule, token-recurrent form, state updated IN PLACE.
 *
 * Replaces the FLA fused_recurrent_gated_delta_rule launch with
 * h0 == ht == initial_state in runtime/model/inference_kernels.py:147-173
 * (called from the decode forward at inference_kernels.py:716) and the torch
 * reference torch_recurrent_gated_delta_rule in the vendored Transformers wheel
 * (transformers/models/qwen3_5/modeling_qwen3_5.py:314-353).
 *
 *   q, k   [B, T, H, K]   (qkv_dtype)
 *   v      [B, T, HV, V]  (qkv_dtype)
 *   g      [B, T, HV]     (g_dtype)     log-decay, state *= exp(g)
 *   beta   [B, T, HV]     (beta_dtype)
 *   state  [n_state_rows, HV, K, V] float32, read and written in place
 *   state_indices  NULL, or int32 [B]: batch row b uses state row
 *                  state_indices[b]; a negative index skips the row (its
 *                  output is zero and no state is touched)
 *   o      [B, T, HV, V]  (qkv_dtype)
 *   scale  multiplier applied to q after the optional L2 normalisation
 *          (the reference uses K ** -0.5)
 *   use_qk_l2norm  nonzero: q and k are L2-normalised over K (eps 1e-6 inside
 *          the rsqrt) before use, as use_qk_l2norm_in_kernel=True
 * Requirements: HV % H == 0; K in {64, 128}; V in {64, 128}; without
 * state_indices, n_state_rows >= B.
 */
int yh_gdn_recurrent(const void* q, const void* k, const void* v, const void* g,
                     const void* beta, float* state, const int32_t* state_indices,
                     void* o, int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K,
                     int64_t V, int64_t n_state_rows, float scale, int use_qk_l2norm,
                     int qkv_dtype, int g_dtype, int beta_dtype, yh_stream_t stream);

/*
 * Packed-varlen form of yh_gdn_recurrent: n_seqs sequences concatenated on one
 * token axis, sequence b owning tokens [cu_seqlens[b], cu_seqlens[b + 1]).
 * q, k [total, H, K]; v, o [total, HV, V]; g, beta [total, HV]; state
 * [n_state_rows, HV, K, V] fp32 in place (row b, or state_indices[b]).
 * Replaces the cu_seqlens form of the FLA call mirrored at
 * runtime/model/inference_kernels.py:147 and the per-request prefill loop of
 * the vLLM adapter (vllm_yanchor.py:85-96).
 */
int yh_gdn_recurrent_varlen(const void* q, const void* k, const void* v, const void* g, const void* beta,
                            float* state, const int32_t* state_indices, const int32_t* cu_seqlens, void* o,
                            int64_t n_seqs, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t n_state_rows,
                            float scale, int use_qk_l2norm, int qkv_dtype, int g_dtype, int beta_dtype,
                            yh_stream_t stream);

/*
 * One decode token of a GDN layer's core in one launch: yh_gdn_decode_prep
 * (conv window update + SiLU, beta, g), yh_gdn_recurrent (T = 1, L2-normed q/k,
 * state IN PLACE) and yh_gated_rmsnorm of the output, bit for bit what those
 * three give with the recurrence at its 128-column tile.
 *
 *   proj [B, proj_stride] bf16: qkv (conv_dim) | ... with z at z_offset
 *        (HV * V), b at b_offset (HV), a at a_offset (HV)
 *   conv_state [B, 3, conv_dim] bf16 (oldest first), shifted in place
 *   conv_w [conv_dim, 4] bf16;  a_log, dt_bias float [HV]
 *   state [n_state_rows, HV, K, V] of state_dtype (row b, or
 *        state_indices[b]; a negative index leaves the state alone and gives
 *        a zero output row before the norm): YH_F32, or YH_F16 for the
 *        reference's fp16 state storage (inference_kernels.py:1079-1081,
 *        modeling_yanchor.py:733-750: widened on the load, the update in fp32,
 *        rounded to nearest on the store)
 *   norm_w [V] bf16;  y [B, HV * V] bf16 = gated RMSNorm (eps) of o with z
 * Requirements: H == HV, K == V == 128, conv_dim == 2 H K + HV V, conv kernel 4;
 * proj rows and z_offset multiples of 4 elements.
 * Replaces the decode-step conv update, fused_recurrent_gated_delta_rule and
 * gated norm of a linear-attention layer (runtime/model/inference_kernels.py:
 * 339-376, 668-716; transformers wheel, qwen3_5 Qwen3_5RMSNormGated 175-190)
 * for the decode graph (no reference counterpart as one launch).
 */
int yh_gdn_decode_fused(const void* proj, int64_t proj_stride, void* conv_state, const void* conv_w,
                        const float* a_log, const float* dt_bias, void* state, int state_dtype,
                        const int32_t* state_indices,
                        const void* norm_w, void* y, int64_t B, int64_t H, int64_t HV, int64_t K, int64_t V,
                        int64_t conv_dim, int64_t z_offset, int64_t b_offset, int64_t a_offset,
                        int64_t n_state_rows, float scale, int use_qk_l2norm, float eps, yh_stream_t stream);

/*
 * Chunked packed-varlen prefill of the gated delta rule on bf16 MFMA (chunk 64).
 *
 * Replaces FLA chunk_gated_delta_rule with cu_seqlens (bound at
 * modeling_yanchor.py:397, 403; called at transformers wheel
 * models/qwen3_5/modeling_qwen3_5.py:519-529) and follows
 * torch_chunk_gated_delta_rule (same file, 234-311).
 *
 *   q, k [total_tokens, H, 128] bf16; v, o [total_tokens, HV, V] bf16 (V 64 or
 *   128; q, k, v and o 16-byte aligned); g, beta [total_tokens, HV] (f32 / bf16
 *   / f16); cu_seqlens int32
 *   [n_seqs + 1] (cu_seqlens[n_seqs] <= total_tokens)
 *   initial_state NULL (zeros) or fp32 [n_seqs, HV, 128, V] (read only)
 *   final_state fp32 [n_seqs, HV, 128, V] (written)
 *   order NULL or int32 [n_seqs]: dispatch order of the sequences (longest
 *   first balances the grid); every sequence must appear once.
 *   workspace, workspace_bytes: unused (may be NULL / 0); every per-chunk
 *   quantity stays on chip.  yh_gdn_chunk_workspace_bytes returns 0.
 *   One launch: a workgroup per (sequence, value head) prepares each chunk
 *   (norms, decays, K K^T, Q K^T, the inverse of I + L) while it runs the
 *   state-dependent products of the previous one.
 */
int yh_gdn_chunk_varlen(const void* q, const void* k, const void* v, const void* g, const void* beta,
                        const float* initial_state, float* final_state, void* o, const int32_t* cu_seqlens,
                        const int32_t* order, int64_t n_seqs, int64_t total_tokens, int64_t H, int64_t HV,
                        int64_t K, int64_t V, float scale, int use_qk_l2norm, int qkv_dtype, int g_dtype,
                        int beta_dtype, void* workspace, int64_t workspace_bytes, yh_stream_t stream);
int64_t yh_gdn_chunk_workspace_bytes(int64_t total_tokens, int64_t n_seqs, int64_t HV, int64_t V);

/*
 * Anchor memory, decode read of the committed slots.
 *
 * Replaces committed_gqa (_read_parts + _read_reduce) in
 * runtime/model/independent_memory.py:47-88, 177-188 and the torch branch of
 * IndependentGQAMemory._decode, modeling_yanchor.py:283-290.
 *
 *   query      [B, H, D]   (dtype)     H = G * R, head h reads group h / R
 *   keys, values [NB, G, capacity, D] (dtype)
 *   positions  [NB, G, capacity] int32, slot live iff >= 0
 *   indices    NULL or int32 [B]: row b reads state row indices[b]; < 0 reads
 *              nothing (output 0)
 *   out        [B, H, D]   (dtype)
 *   keys_row_stride, values_row_stride, positions_row_stride
 *              elements between consecutive state rows; 0 = dense
 *              (G * capacity * D, G * capacity).  Larger strides address a
 *              state inside slot pages, e.g. the vLLM wire format
 *              (vllm_yanchor.py:21-24, 49-64).
 * Per head: out = softmax([q.K^T / sqrt(D) over live slots, 0]) . [V; 0] (a
 * sink logit of 0 with value 0), accumulated in fp32.
 * Requirements: D in {64, 128}; H / G in {1, 2, 4}; capacity a multiple of 16,
 * at most 1024; 16-byte aligned query/keys/values rows.
 */
int yh_anchor_read(const void* query, const void* keys, const void* values, const int32_t* positions,
                   const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t capacity,
                   int64_t D, int64_t n_state_rows, int64_t keys_row_stride, int64_t values_row_stride,
                   int64_t positions_row_stride, int dtype, yh_stream_t stream);

/*
 * Decode attention of one query token over a physical ring of `window` cached
 * key/value slots: the read of yh_anchor_read without the sink (plain softmax
 * over the live slots; no live slot gives 0).  positions [NB, G, window] int32
 * marks live slots (>= 0).  Replaces the physical-ring SWA decode attention
 * (fixed_memory_physical_ring_decode_attention, runtime/model/
 * inference_kernels.py:1881-1898) for D in {64, 128}, H / G in {1, 2, 4} and a
 * window that is a multiple of 16, at most 1024.  Key and value rows are
 * fetched only for blocks of 16 (or 32) slots that hold a live slot, so a ring
 * that fills from slot 0 costs in proportion to its live slots; the result is
 * that of the full pass.
 */
int yh_window_attend(const void* query, const void* keys, const void* values, const int32_t* positions,
                     const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t window, int64_t D,
                     int64_t n_state_rows, int dtype, yh_stream_t stream);

/*
 * yh_anchor_read / yh_window_attend with the decode layer's epilogue applied to
 * the read (each product rounded to the dtype, as the torch ops that follow the
 * read in the reference's decode layer):
 *   anchor_read_gated:  out = (read * row_valid[b]) * head_gate[b, h]
 *                       (modeling_yanchor.py:283-290 read, then the read gate
 *                       of _query_scores 167-176 applied by the caller)
 *   window_attend_gated: out = read * sigmoid(gate[b, h, :])  (the gated-q
 *                       output of the SWA layer, inference_kernels.py:1899-1915)
 * row_valid uint8 [B] (NULL = all valid); head_gate float [B, H] (NULL = 1);
 * gate: rows gate_tok_stride, heads gate_head_stride elements apart, query dtype.
 */
int yh_anchor_read_gated(const void* query, const void* keys, const void* values, const int32_t* positions,
                         const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t capacity,
                         int64_t D, int64_t n_state_rows, int64_t keys_row_stride, int64_t values_row_stride,
                         int64_t positions_row_stride, const uint8_t* row_valid, const float* head_gate, int dtype,
                         yh_stream_t stream);
int yh_window_attend_gated(const void* query, const void* keys, const void* values, const int32_t* positions,
                           const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t window,
                           int64_t D, int64_t n_state_rows, const void* gate, int64_t gate_tok_stride,
                           int64_t gate_head_stride, int dtype, yh_stream_t stream);

/*
 * Anchor memory, decode push and Top-K commit, IN PLACE on the memory state.
 *
 * Replaces commit_decode (_push_select, _gather_commit, _write_commit,
 * _advance) in runtime/model/independent_memory.py:90-175, 190-201 and the
 * torch branch modeling_yanchor.py:291-312.
 *
 *   key, value  [B, G, D] (dtype), batch rows key_row_stride / value_row_stride
 *               elements apart (<= 0: G * D, dense);  score [B, G] float32;
 *               active uint8/bool [B]
 *   indices     NULL or int32 [B] (row -> state row; < 0 skips the row)
 *   keys, values [NB, G, capacity, D]; scores float [NB, G, capacity];
 *   positions int32 [NB, G, capacity]; pending_keys, pending_values
 *   [NB, G, pending_capacity, D]; pending_scores float [NB, G, pending_capacity];
 *   count, total int64 [NB]
 * For each active row with state row b and c = count[b]: (key, value, score)
 * goes to pending slot c; if c + 1 == chunk, every group keeps the best
 * `capacity` of its capacity committed + chunk pending candidates, ordered by
 * score descending, then position ascending (empty slots last), then candidate
 * index (committed 0..capacity-1, then pending 0..chunk-1); pending j has
 * position total[b] - c + j.  Then count = (c + 1) mod chunk and total += 1.
 * row_strides  NULL (dense state) or 9 int64: elements between consecutive
 *   state rows of keys, values, scores, positions, pending_keys,
 *   pending_values, pending_scores, count, total (the IndependentMemoryState
 *   field order), for a state inside slot pages such as the vLLM wire format
 *   (vllm_yanchor.py:21-24, 49-64).
 * Requirements: 1 <= chunk <= pending_capacity; capacity + chunk <= 2048;
 * D * element size a multiple of 16 and capacity * D * element size <= 128 KiB;
 * no state row may appear twice in one call.
 */
int yh_anchor_commit(const void* key, const void* value, const float* score, const uint8_t* active,
                     const int32_t* indices, void* keys, void* values, float* scores, int32_t* positions,
                     void* pending_keys, void* pending_values, float* pending_scores, int64_t* count,
                     int64_t* total, int64_t B, int64_t G, int64_t capacity, int64_t pending_capacity,
                     int64_t chunk, int64_t D, int64_t n_state_rows, const int64_t* row_strides,
                     int64_t key_row_stride, int64_t value_row_stride, int dtype, yh_stream_t stream);

/*
 * Anchor memory, prefill read: each query of a C-token block attends over the
 * source tokens the block references, with the zero-logit sink.
 *
 * Replaces indexed_gqa / _indexed_forward (runtime/model/independent_memory.py:
 * 6-45) and indexed_gqa_torch / _gqa_tile (modeling_yanchor.py:22-42), called
 * from IndependentGQAMemory._sequence (modeling_yanchor.py:249).
 *
 *   query       [B, NB, C, H, D] (dtype)
 *   key, value  [KB, S, G, D]    (dtype); KB == B, or 1 (shared by all rows)
 *   references  [B, NB, G, CAP]  int32 or int64 (ref_dtype): row of S, -1 = none
 *   out         [B, NB, C, H, D]
 * Query head h reads group h / (H / G): out = softmax([q.K^T / sqrt(D), 0]) V
 * over the referenced rows (an index outside [0, S) counts as none).
 * Requirements: D == 128; dtype bf16 or fp16 (YH_ERR_UNSUPPORTED otherwise).
 */
int yh_indexed_gqa(const void* query, const void* key, const void* value, const void* references, int ref_dtype,
                   void* out, int64_t B, int64_t NB, int64_t C, int64_t H, int64_t G, int64_t D, int64_t KB,
                   int64_t S, int64_t CAP, int dtype, yh_stream_t stream);

/*
 * The read of a prefill chunk that continues an anchor-memory state (the
 * block read of IndependentGQAMemory._sequence, modeling_yanchor.py:249, as
 * yh_indexed_gqa) with the tokens addressed in place: query and out are the
 * chunk's tokens [B, L, H, D]; block position p = nb * C + t of row b holds
 * token p - first[b] (first: the row's pending count before the chunk, int64
 * [B]); positions without a token are not read and nothing is written for
 * them.  key, value [B, S, G, D]; references [B, NB, G, CAP] as in
 * yh_indexed_gqa.  No separate counterpart in the reference: it is that read
 * without the block-padded copy of the queries and the gather of the output.
 */
int yh_anchor_sequence_read(const void* query, const void* key, const void* value, const void* references,
                            int ref_dtype, const int64_t* first, void* out, int64_t B, int64_t L, int64_t NB,
                            int64_t C, int64_t H, int64_t G, int64_t D, int64_t S, int64_t CAP, int dtype,
                            yh_stream_t stream);

/*
 * Anchor memory, prefill continuation, step 1: the block-wise Top-K scan of
 * IndependentGQAMemory._sequence with a state (modeling_yanchor.py:178-275:
 * exclusive_prefix_topk 65-78 on the new blocks, merged with the committed
 * slots at 217-219; the state update 256-274).
 *
 * A row's sequence is its old pending tokens (count[b] of them) followed by
 * its counts[b] valid new tokens, cut into blocks of `chunk`.  Source rows of
 * row b: [0, capacity) committed slot, [capacity, capacity + chunk) old
 * pending slot, capacity + chunk + i new token i.
 *
 *   new_scores  [B, L, G] float32, valid tokens first; counts int64 [B]
 *   scores [B, G, capacity] f32, positions [B, G, capacity] i32,
 *   pending_scores [B, G, pending_capacity] f32, count / total int64 [B]
 *               -- the state, dense; scores, positions and pending_scores
 *               are rewritten IN PLACE with the final memory and pending tail
 *   block_refs  [B, NB, G, capacity] int32 out: source rows of the memory in
 *               force for block j (-1 = empty slot)
 *   final_refs  [B, G, capacity] int32 out: source rows of the final memory
 *   pending_refs [B, G, pending_capacity] int32 out: source rows of the new
 *               pending tokens (-1 past the tail)
 * Requirements: chunk <= pending_capacity, chunk <= 1024,
 * capacity + chunk <= 2048, NB * chunk >= L + chunk - 1.  A row whose count is
 * outside [0, chunk) reads nothing (block_refs -1) and keeps its state.
 */
int yh_anchor_prefix(const float* new_scores, const int64_t* counts, float* scores, int32_t* positions,
                     float* pending_scores, const int64_t* count, const int64_t* total, int32_t* block_refs,
                     int32_t* final_refs, int32_t* pending_refs, int64_t B, int64_t L, int64_t G, int64_t capacity,
                     int64_t pending_capacity, int64_t chunk, int64_t NB, yh_stream_t stream);

/*
 * Anchor memory, prefill continuation, step 2: copy the key / value rows of
 * the final memory and the pending tail out of the assembled sources into the
 * state (zeros where a slot references nothing), then count = (count +
 * counts) % chunk, total += counts (modeling_yanchor.py:256-274).
 *
 *   src_keys, src_values [B, S, G, D] (dtype): the source rows above,
 *               S = capacity + chunk + L
 *   final_refs, pending_refs, counts: as written / read by yh_anchor_prefix
 *   keys, values [B, G, capacity, D]; pending_keys, pending_values
 *   [B, G, pending_capacity, D]; count, total int64 [B] -- updated IN PLACE
 */
int yh_anchor_sequence_commit(const void* src_keys, const void* src_values, const int32_t* final_refs,
                              const int32_t* pending_refs, const int64_t* counts, void* keys, void* values,
                              void* pending_keys, void* pending_values, int64_t* count, int64_t* total, int64_t B,
                              int64_t S, int64_t L, int64_t G, int64_t capacity, int64_t pending_capacity,
                              int64_t chunk, int64_t D, int dtype, yh_stream_t stream);

/*
 * Skinny bf16 projection of the decode step: out[M, N] = x[M, K] . W[N, K]^T,
 * fp32 accumulation, bf16 output (torch.nn.functional.linear without bias, the
 * q/k/v/z/b/a, output, MLP, memory-writer and lm_head projections of
 * modeling_yanchor.py:147-176, 877-964 and the Qwen3.5 layers in the
 * transformers wheel) for M <= 128 rows.
 *
 *   x    [M, K] bf16, rows x_stride elements apart (16-byte aligned rows)
 *   w    [N, K] bf16, dense
 *   out  [M, N] bf16, rows out_stride elements apart
 *   split_k    K is split over this many workgroups per 64-column tile
 *              (yh_linear_split gives the library's choice); with
 *              split_k > 1 the partial sums go through `workspace`, which must
 *              hold yh_linear_workspace_bytes(M, N, K, split_k) bytes (16-byte
 *              aligned); a second kernel sums the partials in a fixed order,
 *              so results are identical from call to call.  Calls sharing a
 *              workspace must not overlap.
 * Requirements: 0 <= M <= 128; N % 64 == 0; K % 64 == 0.
 */
int yh_linear(const void* x, int64_t x_stride, const void* w, void* out, int64_t out_stride, int64_t M, int64_t N,
              int64_t K, int64_t split_k, void* workspace, int64_t workspace_bytes, yh_stream_t stream);
int yh_linear_split(int64_t M, int64_t N, int64_t K);
int64_t yh_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t split_k);

/*
 * The same projection with the weights repacked once into MFMA fragment order
 * (no counterpart in the reference, which keeps nn.Linear weights row-major;
 * the packed copy serves the decode step, the row-major one everything else).
 *
 * yh_linear_pack: w [N, K] bf16 row-major -> packed [N * K] bf16 with
 *   packed[((kb * N/16 + T) * 64 + l) * 8 + e] = w[16 T + l % 16][32 kb + 8 (l / 16) + e]
 *   (column tile T of 16 outputs, K block kb of 32; lane l of a 16x16x32 MFMA
 *   B operand; K blocks outermost since ABI 104, tile-major before).
 *   N % 16 == 0, K % 32 == 0.  With pair_halves the tiles
 *   alternate between the row halves of w (tile 2j = rows 16j.., tile 2j+1 =
 *   rows N/2 + 16j..; N % 32 == 0): the layout of a [gate; up] MLP weight for
 *   the silu epilogue.
 * yh_linear_packed: out[M, N] = x[M, K] . W^T from the packed weights; split_k
 *   slices K in whole 128-wide phases (yh_linear_packed_split gives the
 *   library's choice); with more than one slice the workspace must hold
 *   split_k * M * N * 4 bytes (16-byte aligned) and the partial sums are added
 *   in a fixed order.  residual (NULL = none) [M, N] bf16, rows residual_stride
 *   apart: out = bf16(bf16(x . W^T) + residual), the decode layers'
 *   `z = x + proj(...)` adds (modeling_yanchor.py:159, 903-905).  silu_pairs
 *   (weights packed with pair_halves, split_k == 1, no residual): out is
 *   [M, N/2] = bf16(bf16(silu(gate)) * up), the MLP activation
 *   (inference_kernels.py:642-666) in the projection's store.  The work
 *   split (columns per workgroup, waves) is yh_proj_pick's for the shape;
 *   the output rows (and the residual's) are written 16 bytes at a time and
 *   must be 16-byte aligned.
 *   Requirements: 0 <= M <= 256 (past 128 rows, one configuration with
 *   256-row tiles), N % 16 == 0, K % 128 == 0.
 */
int yh_linear_pack(const void* w, void* packed, int64_t N, int64_t K, int pair_halves, yh_stream_t stream);
int yh_linear_packed(const void* x, int64_t x_stride, const void* w_packed, void* out, int64_t out_stride, int64_t M,
                     int64_t N, int64_t K, const void* residual, int64_t residual_stride, int silu_pairs,
                     int64_t split_k, void* workspace, int64_t workspace_bytes, int defer_reduce,
                     int64_t* slices_out, yh_stream_t stream);
int yh_linear_packed_split(int64_t M, int64_t N, int64_t K);

/* Sampling semantics of yh_topk_sample. */
enum yh_sample_mode {
  /* _qwen35_top20_counter_sample_kernel (runtime/model/inference_kernels.py:
   * 1119-1145): softmax of the top-k after temperature, keep p where the mass
   * before it is < top_p, u unclamped, rank = #(cumulative < u * retained). */
  YH_SAMPLE_FUSED = 0,
  /* sample_top_k_top_p_counter (inference_kernels.py:35-88): the same
   * truncation, renormalised, u clamped below 1, threshold
   * min(u * total, nextafter(total, 0)), searchsorted left. */
  YH_SAMPLE_TORCH = 1
};

/*
 * Top-k / top-p counter sampling of one token per row, with the dense presence
 * penalty fused in (scores are not modified).
 *
 * Replaces torch.topk + _qwen35_top20_counter_sample_kernel
 * (_sample_top_k_top_p_counter_triton, runtime/model/inference_kernels.py:
 * 1147-1167) and sample_top_k_top_p_counter (inference_kernels.py:73-88).
 * Both modes take 1 <= top_k <= 64.  The torch-sampler mode also takes the
 * reference's other branches (inference_kernels.py:78-86): top_k <= 0 with
 * top_p == 1 draws from the softmax over the whole vocabulary in vocabulary
 * order; top_k <= 0 (the whole vocabulary) or top_k > 64 with any top_p
 * keeps the top k by value and truncates at top_p.  Those run one workgroup
 * per row with exact fixed-point probability sums, need no workspace (it may
 * be NULL) and return no top-k values.
 *
 *   scores       [B, V] rows `row_stride` elements apart (f32 / bf16 / f16)
 *   seen         NULL or uint8/bool [B, V] rows `seen_stride` apart; where set,
 *                `penalty` is subtracted from the score before selection
 *   attempt_ids  int64 [B]; steps int64 [B] or NULL (then `step` for all rows)
 *   seed, stream_id  counter-hash seed and stream (taken mod 2^32)
 *   tokens       int64 [B] output
 *   out_values, out_indices  NULL or [B, top_k] float / int64: the selected
 *                top-k (descending; equal values by ascending index)
 *   workspace    device scratch of at least yh_topk_workspace_bytes(B, V, k)
 *                (1 <= k <= 64)
 * top_k == 1 returns the argmax.  Otherwise temperature > 0, 0 < top_p <= 1.
 */
int yh_topk_sample(const void* scores, int dtype, int64_t row_stride, const uint8_t* seen, int64_t seen_stride,
                   float penalty, const int64_t* attempt_ids, const int64_t* steps, int64_t step, uint64_t seed,
                   uint64_t stream_id, float temperature, int64_t top_k, float top_p, int mode, int64_t* tokens,
                   float* out_values, int64_t* out_indices, void* workspace, int64_t workspace_bytes, int64_t B,
                   int64_t V, yh_stream_t stream);

/* Workspace bytes yh_topk_sample needs, and its vocabulary split into
 * 8192-element segments (bf16 rows of 16-byte runs with top_k <= 32 take half
 * as many segments of 16384, within the same workspace). */
int64_t yh_topk_workspace_bytes(int64_t B, int64_t V, int64_t top_k);
void yh_topk_segments(int64_t V, int64_t top_k, int* n_segments, int* seg_len);

/*
 * yh_topk_sample without a workspace argument: it allocates nothing and calls
 * no allocating routine.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, kernels and results as yh_topk_sample.  The candidate lists
 * live in a static device array of YH_TOPK_STATIC_SCRATCH_BYTES per GPU
 * (8 MiB, held until the process ends); calls whose yh_topk_workspace_bytes
 * (B, V, top_k) exceed it return YH_ERR_INVALID.  At V = 151936 that is up to
 * 2759 rows at top_k = 20, 862 rows at top_k = 64.  The stream's device must
 * be the current device.  Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams, other host threads) race.
 */
#define YH_TOPK_STATIC_SCRATCH_BYTES (8ll << 20)
int yh_topk_sample_noalloc(const void* scores, int dtype, int64_t row_stride, const uint8_t* seen,
                           int64_t seen_stride, float penalty, const int64_t* attempt_ids, const int64_t* steps,
                           int64_t step, uint64_t seed, uint64_t stream_id, float temperature, int64_t top_k,
                           float top_p, int mode, int64_t* tokens, float* out_values, int64_t* out_indices,
                           int64_t B, int64_t V, yh_stream_t stream);

/*
 * scores[i] -= penalty where seen[i], float32, in place; n elements.
 * Replaces _qwen35_dense_presence_penalty_kernel / _apply_dense_presence_penalty_
 * (runtime/model/inference_kernels.py:1095-1114).
 */
int yh_presence_penalty(float* scores, const uint8_t* seen, int64_t n, float penalty, yh_stream_t stream);

/*
 * u = float32((hash + 0.5) / 2^32), clamped below 1, for n counters
 * (attempt_ids[i], steps ? steps[i] : step, seed, stream_id).
 * Replaces counter_uniform (runtime/model/inference_kernels.py:24-33).
 */
int yh_counter_uniform(const int64_t* attempt_ids, const int64_t* steps, int64_t step, uint64_t seed,
                       uint64_t stream_id, float* out, int64_t n, yh_stream_t stream);

/*
 * Per-step slot bookkeeping after sampling, for all `slots` rows:
 *   active = !finished[r] && slot_rows[r] >= 0
 *   storage[active ? slot_rows[r] : sink_rows[r], active ? row_steps[r] :
 *           maximum_new_tokens] = active ? token : pad
 *   dense_seen[r, stored] = 1; generated_lengths / finished_by_eos of the
 *   written row; finished[r] |= active && (eos || steps >= cap);
 *   row_steps[r] += active; row_positions[r] += active;
 *   decode_ids[r] = finished ? pad : stored; *decode_useful_events += #active.
 * Replaces _qwen35_decode_state_update_kernel / _update_fixed_decode_state_
 * (runtime/model/inference_kernels.py:1169-1208).
 * Types: sampled_token, decode_ids int64 [slots] (the [slots, 1] token
 * tensors); storage int32 [storage_rows, storage_width]; dense_seen bool
 * [slots, seen_width]; generated_lengths int64 and finished_by_eos bool
 * [storage_rows]; finished bool and slot_rows, sink_rows, slot_caps, row_steps,
 * row_positions int64 [slots]; decode_useful_events int64 scalar.
 * eos_token_ids is a HOST array of eos_count ids (the first two are used).
 * Stores that would fall outside their tensor are skipped.
 */
int yh_decode_bookkeeping(const int64_t* sampled_token, int32_t* storage, uint8_t* dense_seen,
                          int64_t* generated_lengths, uint8_t* finished_by_eos, uint8_t* finished,
                          const int64_t* slot_rows, const int64_t* sink_rows, const int64_t* slot_caps,
                          int64_t* row_steps, int64_t* row_positions, int64_t* decode_ids,
                          int64_t* decode_useful_events, int64_t slots, int64_t storage_rows, int64_t storage_width,
                          int64_t seen_width, int64_t maximum_new_tokens, int64_t pad_token_id,
                          const int64_t* eos_token_ids, int64_t eos_count, yh_stream_t stream);

/*
 * cu_seqlens[0] = 0, cu_seqlens[i + 1] = sum(lengths[:i + 1]) (int32 out,
 * lengths int32 or int64, n sequences): the packed-varlen offsets consumed by
 * the chunked prefill (the cu_seqlens argument mirrored at
 * runtime/model/inference_kernels.py:147; vLLM's query_start_loc,
 * vllm_yanchor.py:85-96).
 */
int yh_cu_seqlens(const void* lengths, int lengths_dtype, int32_t* cu_seqlens, int64_t n, yh_stream_t stream);

enum yh_select_mode {
  YH_SELECT_KEEP = 0,     /* !finished && slot_rows >= 0: tail-compaction keep-list
                             (torch.nonzero at runtime/model/inference_kernels.py:1725) */
  YH_SELECT_FINISHED = 1  /* finished: refill targets (inference_kernels.py:1549) */
};

/*
 * Ascending indices i < n that satisfy the mode's predicate into out[0..count),
 * out[count..n) = -1, *count (device int64) = number selected.
 */
int yh_select_slots(const uint8_t* finished, const int64_t* slot_rows, int mode, int64_t* out, int64_t* count,
                    int64_t n, yh_stream_t stream);

/*
 * For each of n_tensors tensors t (host arrays of device pointers and sizes):
 * dst[t][dst_index[i]] = src[t][src_index[i]] for i < n, rows of row_bytes[t]
 * bytes; a NULL index array means the identity.  Indices outside
 * [0, src_rows[t]) / [0, dst_rows[t]) are skipped.  src[t] and dst[t] must be
 * different buffers.  The row ops of the fixed-memory caches:
 * batch_select_indices / batch_scatter_from (modeling_yanchor.py:540-554,
 * 647-683, 723-731).
 */
int yh_gather_rows(int n_tensors, const void* const* src, void* const* dst, const int64_t* row_bytes,
                   const int64_t* src_rows, const int64_t* dst_rows, const int64_t* src_index,
                   const int64_t* dst_index, int64_t n, yh_stream_t stream);

/* ---- fused decode-layer neighbours (bf16 activations) ------------------- */

/*
 * Qwen3.5 RMSNorm over rows of D bf16 values: s = residual ? bf16(x + residual)
 * : x; residual_out (optional) = s; out = bf16(s / sqrt(mean(s^2) + eps) *
 * (plus_one ? 1 + w : w)).  x rows x_stride apart, out rows out_stride apart,
 * residual / residual_out contiguous [N, D].  D % 8 == 0, D <= 8192.
 * Replaces _qwen35_rmsnorm_torch_tree_kernel / the fused residual RMSNorm
 * (runtime/model/inference_kernels.py:227-271, 1767-1797).
 */
int yh_rmsnorm(const void* x, int64_t x_stride, const void* residual, void* residual_out, const void* w, void* out,
               int64_t out_stride, int64_t N, int64_t D, float eps, int plus_one, yh_stream_t stream);

/*
 * Inputs of one decode step, one launch: h = embed[tokens] (bf16 [B, D]; a
 * zero row for an id outside [0, V)), xn = RMSNorm(h) * (1 + w) as yh_rmsnorm,
 * cos / sin float [B, rotary_dim] of float(positions[b]) * inv_freq[j mod
 * rotary_dim / 2] (rotate-half layout; inv_freq float [rotary_dim / 2]), the
 * SWA ring row ring_rows[b] = b * ring_stride + positions[b] mod window, and,
 * when finished (bool [B]), slot_rows (int64 [B]) and valid (bool [B]) are all
 * given, valid[b] = !finished[b] && slot_rows[b] >= 0.  D % 8 == 0, D <= 8192.
 * Replaces the embedding lookup and rotary tables of the model forward
 * (modeling_yanchor.py:932, 951) and the live-slot mask of the decode step
 * (runtime/model/inference_kernels.py:1176) for the fixed-slot decode graph.
 */
int yh_decode_inputs(const int64_t* tokens, const int64_t* positions, const void* embed, int64_t V, const void* w,
                     const float* inv_freq, const uint8_t* finished, const int64_t* slot_rows, void* h, void* xn,
                     float* cos, float* sin, int64_t* ring_rows, uint8_t* valid, int64_t B, int64_t D,
                     int64_t rotary_dim, int64_t ring_stride, int64_t window, float eps, yh_stream_t stream);

/*
 * yh_rmsnorm whose input row is a split-K projection still in fp32 partials
 * (yh_linear_packed with defer_reduce): x = bf16(sum over the S planes of
 * part [S, N, D] in slice order), x = bf16(x + proj_residual) when given (the
 * projection's own residual add), then as yh_rmsnorm with `residual`.  The
 * projection's residual may instead be a second projection's partials part2
 * [S2, N, D] (ABI 105; NULL = none; not with proj_residual; S + S2 <= 64),
 * summed in slice order and rounded to bf16 first, as a separate reduce would
 * store it: the attention layer's output projection joining the memory
 * output projection without a reduce launch of its own.  With
 * w2 / out2 (both or neither) the same row is also normed with the weight w2
 * into out2 ([N, D], rows out2_stride >= D elements apart; ABI 103 added the
 * stride): the decode layers whose memory path norms the layer input with its
 * own weight.  The reduce of the projection and the
 * norms after it in one launch (no reference counterpart: the reference runs
 * the projection, the adds and each norm as separate ops).
 */
int yh_rmsnorm_partials(const float* part, int64_t S, const void* proj_residual, int64_t proj_residual_stride,
                        const float* part2, int64_t S2, const void* residual, void* residual_out, const void* w,
                        void* out, int64_t out_stride,
                        int64_t N, int64_t D, float eps, int plus_one, const void* w2, void* out2,
                        int64_t out2_stride, yh_stream_t stream);

/*
 * GDN decode prologue for B rows of the packed projection proj [B, proj_stride]
 * (bf16) = [q k v (conv_dim) | z | b (HV) at b_offset | a (HV) at a_offset]:
 * depthwise causal conv1d update with conv_state [B, conv_kernel - 1, conv_dim]
 * (bf16, time-major, shifted in place) and conv_w [conv_dim, conv_kernel], SiLU,
 * split into q, k [B, qk_dim] and v [B, conv_dim - 2 qk_dim] (bf16), and the gates
 * beta = sigmoid(b), g = -exp(a_log) * softplus(a + dt_bias) (float [B, HV]).
 * Replaces _qwen35_graph_safe_conv_update_kernel and
 * _qwen35_fused_gdn_gates_kernel (runtime/model/inference_kernels.py:339-376,
 * 668-691).  conv_kernel must be 4.
 */
int yh_gdn_decode_prep(const void* proj, int64_t proj_stride, void* conv_state, const void* conv_w,
                       const float* a_log, const float* dt_bias, void* q, void* k, void* v, float* g, float* beta,
                       int64_t B, int64_t conv_dim, int64_t qk_dim, int64_t HV, int64_t b_offset, int64_t a_offset,
                       int64_t conv_kernel, yh_stream_t stream);

/*
 * Qwen3_5RMSNormGated per head of D = 128: out = bf16(bf16(w * bf16(o / rms(o)))
 * * silu(z)); o, out [N, H, 128] contiguous bf16, z head h of row n at
 * z + n * z_stride + h * 128.  (transformers wheel
 * models/qwen3_5/modeling_qwen3_5.py:175-190)
 */
int yh_gated_rmsnorm(const void* o, const void* z, int64_t z_stride, const void* w, void* out, int64_t N, int64_t H,
                     int64_t D, float eps, yh_stream_t stream);

/* out[n, i] = bf16(bf16(silu(gu[n, i])) * gu[n, I + i]) for gate_up [N, 2I]
 * (runtime/model/inference_kernels.py:642-666).  I % 8 == 0. */
int yh_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t N, int64_t I, yh_stream_t stream);

/*
 * Per-head RMSNorm (1 + w) and rotate-half RoPE on the first rotary_dim of
 * D = 128 dims, cos / sin float [N, rotary_dim]: head h of token n is read at
 * x + n * x_tok_stride + h * x_head_stride and written at
 * out + r * out_tok_stride + h * out_head_stride with r = out_tok_index ?
 * out_tok_index[n] : n (e.g. a ring slot).  (modeling_yanchor.py:46-49 and the
 * Qwen3.5 attention q / k path)
 */
int yh_head_norm_rope(const void* x, int64_t x_tok_stride, int64_t x_head_stride, const void* w, const float* cos,
                      const float* sin, void* out, int64_t out_tok_stride, int64_t out_head_stride,
                      const int64_t* out_tok_index, int64_t N, int64_t H, int64_t D, int64_t rotary_dim, float eps,
                      yh_stream_t stream);

/*
 * The ring write of a decode token into the SWA cache: head h of key k is
 * normed and rotated as yh_head_norm_rope and written to ring_k, the raw value
 * head to ring_v and positions[n] to ring_pos, all at ring row rows[n]
 * (rows[n] = n * H * window + positions[n] % window for a per-slot ring):
 *   ring_k / ring_v [N, H, window, 128]: element rows[n] * 128 + h * window * 128 + d
 *   ring_pos int32 [N, H, window]:       element rows[n] + h * window
 * (the chrono ring write of runtime/model/inference_kernels.py:1828-1879 with
 * the key path of the Qwen3.5 attention)
 */
int yh_ring_write(const void* k, int64_t k_tok_stride, int64_t k_head_stride, const void* v, int64_t v_tok_stride,
                  int64_t v_head_stride, const void* w, const float* cos, const float* sin, const int64_t* rows,
                  const int64_t* positions, void* ring_k, void* ring_v, int32_t* ring_pos, int64_t N, int64_t H,
                  int64_t window, int64_t D, int64_t rotary_dim, float eps, yh_stream_t stream);

/*
 * The anchor-memory read prologue of one decode token per row
 * (IndependentGQAMemory._query_scores, modeling_yanchor.py:167-176), from the
 * fused projection proj [B, >= feat_offset + A] bf16 whose first H * 128
 * columns are the query heads and columns [feat_offset, feat_offset + A) the
 * admission features:
 *   q      = RoPE(RMSNorm_(1+w)(q_h))                       bf16 [B, H, 128]
 *   gate   = tanh(read_scale) * 2 * sigmoid(<qn_h, gate_w_h> / sqrt(128) + gate_b)
 *            (qn_h the normed, unrotated head as bf16)      float [B, H]
 *   scores = bf16(silu(features)) . adm_up^T                float [B, G]
 *   act    = bf16(bf16(silu(gate)) * up)                    bf16 [B, act_width]
 *            (the writer's activation of _write_kv, modeling_yanchor.py:
 *            159-166: gate = proj columns [act_offset, act_offset + act_width),
 *            up the act_width columns after them; act rows act_stride apart;
 *            act NULL skips it; 16-byte aligned rows)
 * read_scale, gate_b float [H]; gate_w float [H, 128]; adm_up float [G, A].
 */
int yh_memory_prologue(const void* proj, int64_t proj_stride, int64_t feat_offset, const void* q_norm_w,
                       const float* cos, const float* sin, const float* read_scale, const float* gate_w,
                       const float* gate_b, const float* adm_up, void* q, float* gate, float* scores, int64_t B,
                       int64_t H, int64_t D, int64_t G, int64_t A, int64_t rotary_dim, float eps, int64_t act_offset,
                       int64_t act_width, void* act, int64_t act_stride, yh_stream_t stream);

/*
 * Decode projection on packed weights with a selectable work split
 * (configuration `config`, 0 <= config < yh_proj_config_count()): out[M, N] =
 * x[M, K] . W[N, K]^T, M <= 256 (M > 128: configuration 0 only), the weights in yh_linear_pack's fragment
 * order, the epilogues of yh_linear_packed (residual, silu pairs).  No
 * counterpart in the reference: the reference's decode projections are
 * torch.nn.functional.linear calls (modeling_yanchor.py:147-176 and the
 * Qwen3.5 projections of the transformers wheel) and its packed Triton GEMVs
 * (runtime/model/inference_kernels.py:939-1001).  A configuration fixes the
 * columns per workgroup (yh_proj_columns) and the K granularity
 * (yh_proj_phase_k: K and every K slice are multiples of it).  With the K
 * split over S > 1 slices the fp32 partials [S, M, N] go to `workspace` and
 * are summed by yh_linear_reduce or a partial-aware norm; *slices_out
 * receives S.
 */
int yh_proj(const void* x, int64_t x_stride, const void* w_packed, void* out, int64_t out_stride, int64_t M,
            int64_t N, int64_t K, const void* residual, int64_t residual_stride, int silu_pairs, int config,
            int64_t split_k, void* workspace, int64_t workspace_bytes, int64_t* slices_out, yh_stream_t stream);
int yh_proj_config_count(void);
int yh_proj_phase_k(int config);
int yh_proj_columns(int config);
/* The configuration and K split yh_linear_packed uses for a shape (no
 * counterpart in the reference; K a multiple of 128). */
int yh_proj_pick(int64_t M, int64_t N, int64_t K, int silu_pairs, int* config, int64_t* split_k);

/*
 * out[M, N] = bf16(sum over s of part[s]) (+ residual, added to the bf16
 * sum): the split-K reduce of yh_linear_packed / yh_proj, slices added in
 * order.  part fp32 [S, M, N] (16-byte aligned); out rows out_stride apart
 * (out and residual 8-byte aligned, strides multiples of 4 elements).
 */
int yh_linear_reduce(const float* part, void* out, int64_t out_stride, int64_t M, int64_t N, int64_t S,
                     const void* residual, int64_t residual_stride, yh_stream_t stream);

/*
 * Refill prefill of a packed, ragged set of prompt pieces (cu_seqlens int32
 * [n_seqs + 1], empty pieces allowed), each continuing its sequence's caches.
 *
 * yh_conv_prefill: the GDN layer's causal depthwise conv1d (4 taps) + SiLU
 * over every packed token, the causal-conv1d prefill of the CUDA backend
 * (bound at modeling_yanchor.py:392-407; torch form wheel transformers/models/
 * qwen3_5/modeling_qwen3_5.py:455-470).
 *   proj    [total_tokens, >= channels] (row stride proj_stride): the conv
 *           inputs are its first `channels` columns
 *   window  [n_seqs, 3, channels] time-major (oldest first): the inputs before
 *           each piece (zeros for a fresh sequence); on return it holds the
 *           last 3 inputs of [window | piece]
 *   conv_w  [channels, 4]
 *   out     [total_tokens, channels] = bf16(silu(sum_j x(t-3+j) w[c, j])),
 *           fp32 taps in the order of the decode prologue (yh_gdn_decode_prep)
 * dtype: bf16.
 */
int yh_conv_prefill(const void* proj, int64_t proj_stride, void* window, const void* conv_w,
                    const int32_t* cu_seqlens, int64_t n_seqs, int64_t total_tokens, int64_t channels, void* out,
                    int dtype, yh_stream_t stream);

/*
 * yh_swa_prefill: sliding-window causal attention of every packed query over
 * the `window` keys that end at its own position (key position in
 * [p - window + 1, p]), GQA (query head h reads KV head h / (H / G)), with the
 * keys before each piece read from that sequence's physical ring.  Replaces
 * flash_swa (flash_attn_varlen_func with causal=True, window_size=(W - 1, 0))
 * and reference_swa with query_start (modeling_yanchor.py:412-449), as called
 * by Qwen3_5FixedWindowAttention.forward (modeling_yanchor.py:849-870), and the
 * output gate read * sigmoid(gate) (871-875).
 *   q       [total, H, 128] (token stride q_stride elements), normed and rotated
 *   k, v    [total, G, 128] piece keys (normed, rotated) and values
 *   ring_k, ring_v  [ring_batch, G, window, 128]: slot = position % window
 *   ring_rows int64 [n_seqs]: each piece's ring row, -1 = no context (a fresh
 *           sequence); starts int64 [n_seqs]: position of each piece's first
 *           token; the min(start, window - 1) keys before it come from the ring
 *   tiles   int32 [n_tiles, 2]: (piece, first token) of every tile of
 *           64 / (H / G) tokens that covers the pieces
 *   gate    NULL or [total, H, 128] with the given strides: out = bf16(bf16(o)
 *           * bf16(sigmoid(gate)))
 *   out     [total, H, 128]
 * Requirements: D == 128; H / G divides 64; dtype bf16 or fp16
 * (YH_ERR_UNSUPPORTED otherwise); 16-byte aligned rows.
 */
int yh_swa_prefill(const void* q, int64_t q_stride, const void* k, int64_t k_stride, const void* v, int64_t v_stride,
                   const void* ring_k, const void* ring_v, const int64_t* ring_rows, const int64_t* starts,
                   const int32_t* cu_seqlens, const int32_t* tiles, int64_t n_tiles, const void* gate,
                   int64_t gate_token_stride, int64_t gate_head_stride, void* out, int64_t n_seqs,
                   int64_t ring_batch, int64_t H, int64_t G, int64_t D, int64_t window, int dtype,
                   yh_stream_t stream);

/*
 * yh_ring_fill: the last min(window, L) keys, values and positions of each
 * packed piece into its ring row (slot = position % window), the ring a
 * prefill leaves for the decode read (the chronological ring of
 * runtime/model/inference_kernels.py:1799-1856 built in place; pieces with
 * ring_rows[r] < 0 write nothing).  k, v [total, G, 128] with token strides;
 * ring_k / ring_v [ring rows, G, window, 128]; ring_pos int32 [ring rows, G,
 * window].
 */
int yh_ring_fill(const void* k, int64_t k_stride, const void* v, int64_t v_stride, const int64_t* ring_rows,
                 const int64_t* starts, const int32_t* cu_seqlens, int64_t n_seqs, int64_t total_tokens,
                 void* ring_k, void* ring_v, int32_t* ring_pos, int64_t G, int64_t D, int64_t window, int dtype,
                 yh_stream_t stream);

/*
 * HBM calibration stream (no counterpart in the reference: the measuring stick
 * for the HBM-bound kernels, whose roofline fractions are quoted against the
 * 8 TB/s spec figure).  kind 0: dst <- src; 1: dst <- 0.5 dst + 1 in place;
 * 2: read src (dst receives one float per workgroup); 3: dst <- constant.
 * nontemporal selects nontemporal loads and stores.  bytes: a positive
 * multiple of 16; both buffers 16-byte aligned; grid workgroups of 256
 * threads stride over the buffer.
 */
int yh_hbm_stream(int kind, int nontemporal, const void* src, void* dst, int64_t bytes, int grid,
                  yh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* YANCHOR_AMD_H */
