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
 * Per head: out = softmax([q.K^T / sqrt(D) over live slots, 0]) . [V; 0] (a
 * sink logit of 0 with value 0), accumulated in fp32.
 * Requirements: D in {64, 128}; H / G in {1, 2, 4}; capacity a multiple of 64,
 * at most 1024; 16-byte aligned query/keys/values.
 */
int yh_anchor_read(const void* query, const void* keys, const void* values, const int32_t* positions,
                   const int32_t* indices, void* out, int64_t B, int64_t H, int64_t G, int64_t capacity,
                   int64_t D, int64_t n_state_rows, int dtype, yh_stream_t stream);

/*
 * Anchor memory, decode push and Top-K commit, IN PLACE on the memory state.
 *
 * Replaces commit_decode (_push_select, _gather_commit, _write_commit,
 * _advance) in runtime/model/independent_memory.py:90-175, 190-201 and the
 * torch branch modeling_yanchor.py:291-312.
 *
 *   key, value  [B, G, D] (dtype);  score [B, G] float32;  active uint8/bool [B]
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
 * Requirements: 1 <= chunk <= pending_capacity; capacity + chunk <= 2048;
 * D * element size a multiple of 16 and capacity * D * element size <= 128 KiB;
 * no state row may appear twice in one call.
 */
int yh_anchor_commit(const void* key, const void* value, const float* score, const uint8_t* active,
                     const int32_t* indices, void* keys, void* values, float* scores, int32_t* positions,
                     void* pending_keys, void* pending_values, float* pending_scores, int64_t* count,
                     int64_t* total, int64_t B, int64_t G, int64_t capacity, int64_t pending_capacity,
                     int64_t chunk, int64_t D, int64_t n_state_rows, int dtype, yh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* YANCHOR_AMD_H */
