/*
 * nq_attn.h -- C ABI of the MI355X (gfx950) paged attention library
 * (libnq_attn.so).
 *
 * The library replaces the device work of nano_qwen's paged attention path:
 * the Triton KV scatter and flash_attn's prefill/decode calls made by
 * layers/attention.py, and the Triton decode-metadata kernel of
 * engine/decode_init.py.  All entry points:
 *
 *   - take device pointers, plain integers and floats, and a hipStream_t
 *     passed as `void *` (NULL = the default stream); no torch types;
 *   - enqueue work asynchronously on that stream: they never allocate, free
 *     or synchronise, so they may be captured into a HIP graph;
 *   - return NQ_OK (0) or a negative status; nq_last_error() then returns a
 *     message for the calling thread.
 *
 * Element types are NQ_F32 / NQ_F16 / NQ_BF16 / NQ_FP8_E4M3 (OCP e4m3fn).
 * Strides are in elements of the tensor's own type.
 *
 * KV cache layout (engine/model_runner.py:198): one tensor per layer and
 * per K/V, [num_blocks, block_size, num_kv_heads, head_dim], contiguous;
 * cache row `slot` = block * block_size + offset.
 */
#ifndef NQ_ATTN_H
#define NQ_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NQ_ABI_VERSION 1

#define NQ_OK 0
#define NQ_EINVAL (-1)       /* bad pointer, shape, stride or alignment */
#define NQ_EUNSUPPORTED (-2) /* dtype / head_dim / block_size not built */
#define NQ_ELAUNCH (-3)      /* the HIP launch itself failed */

enum nq_dtype { NQ_F32 = 0, NQ_F16 = 1, NQ_BF16 = 2, NQ_FP8_E4M3 = 3 };

/* Version of this ABI (NQ_ABI_VERSION). */
int nq_abi_version(void);

/* Message for the last non-zero status returned on this thread. */
const char *nq_last_error(void);

/*
 * Slot-mapped KV scatter.
 * Replaces store_kvcache / store_kvcache_kernel (layers/attention.py:10-40).
 *
 * For each token i < num_tokens with slot = slot_mapping[i] in
 * [0, num_slots): copy the num_kv_heads*head_dim elements of key row i
 * (at key + i*key_row_stride) to k_cache row `slot`, and likewise value ->
 * v_cache.  slot == -1 (and any slot outside [0, num_slots)) skips the token,
 * as the reference skips -1 (:23).  key/value rows must be contiguous over
 * (head, dim) -- the reference asserts stride(1) == head_dim and
 * stride(-1) == 1 (:36-37).
 *
 * in_dtype == cache_dtype: a byte-exact copy.
 * cache_dtype == NQ_FP8_E4M3 (in_dtype F32/F16/BF16): each element x of kv
 * head h is stored as e4m3fn(RNE(clamp(float(x) * (1.0f / scale[h]), +-448)))
 * with k_scale / v_scale float[num_kv_heads] device arrays.
 */
int nq_store_kvcache(const void *key, int64_t key_row_stride,
                     const void *value, int64_t value_row_stride,
                     void *k_cache, void *v_cache,
                     const int32_t *slot_mapping, int64_t num_tokens,
                     int64_t num_slots, int num_kv_heads, int head_dim,
                     int in_dtype, int cache_dtype,
                     const float *k_scale, const float *v_scale,
                     void *stream);

/*
 * Split plan for nq_paged_decode, chosen from host-known shapes only (so it
 * is fixed under graph capture): fills *num_splits and *split_tokens (a
 * multiple of 128; split s covers tokens [s*split_tokens, (s+1)*split_tokens)).
 * A multi-split plan for a kernel with one resident workgroup per CU (fp8
 * caches with >= 8 kv heads) may carry more splits than the table needs:
 * the workspace sized from them then also holds the stream-K partials, and
 * nq_paged_decode splits the batch's tokens into equal per-CU ranges instead
 * (NQ_DECODE_STREAMK=0 keeps split-K; nq_decode_schedule tells which).
 */
int nq_decode_plan(int batch, int num_q_heads, int num_kv_heads,
                   int max_blocks_per_seq, int block_size, int kv_dtype,
                   int *num_splits, int *split_tokens);

/* Bytes of device workspace nq_paged_decode needs for a plan (0 if one split). */
int64_t nq_decode_workspace_bytes(int batch, int num_q_heads, int head_dim,
                                  int num_splits);

/*
 * Which multi-split schedule nq_paged_decode takes for these shapes, plan
 * and workspace size: 1 = stream-K (equal per-CU token ranges and a
 * boundary-searched merge), 0 = split-K (or a single split); negative on
 * bad arguments.  No counterpart in the reference (flash_attn picks its
 * split internally); it exists so tests and tuning can tell which path a
 * launch ran.  Stream-K needs a multi-split plan, a kernel with one resident
 * workgroup per CU, a workspace that holds its partials, at most 4096
 * sequences, and batch x table tokens below 2^31 that fit 65535 ranges of
 * 61 blocks; NQ_DECODE_STREAMK=0 forces split-K.  Needs a current device.
 */
int nq_decode_schedule(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                       int max_blocks_per_seq, int block_size, int kv_dtype,
                       int num_splits, int64_t workspace_bytes);

/*
 * Paged decode attention (one query token per sequence).
 * Replaces flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 *   cache_seqlens=context_lens, block_table=block_tables,
 *   softmax_scale=scale, causal=True)   (layers/attention.py:71-74).
 *
 * head_dim is 128 or 256 (NQ_EUNSUPPORTED otherwise).
 * q   [batch, num_q_heads, head_dim] with strides (q_batch_stride,
 *     q_head_stride, 1); out likewise.  q and out have type q_dtype
 *     (F16/BF16).  k_cache/v_cache have type kv_dtype (== q_dtype, or
 *     NQ_FP8_E4M3 with k_scale/v_scale float[num_kv_heads]).
 * block_tables [batch, >= max_blocks_per_seq] int32 with row stride
 * bt_stride; context_lens [batch] int32 counts the cached tokens including
 * the one just stored.  Query head h reads kv head h / (num_q_heads /
 * num_kv_heads).  Entries past ceil(context_len / block_size) are never
 * read; rows with context_len <= 0 produce zeros.
 * num_splits/split_tokens come from nq_decode_plan; workspace (>=
 * nq_decode_workspace_bytes, 256-byte aligned) is caller-owned.  Results do
 * not depend on which of the two multi-split schedules runs beyond float32
 * rounding of the merge.
 */
int nq_paged_decode(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                    const void *k_cache, const void *v_cache,
                    const int32_t *block_tables, int64_t bt_stride,
                    int max_blocks_per_seq, const int32_t *context_lens,
                    void *out, int64_t out_batch_stride, int64_t out_head_stride,
                    int batch, int num_q_heads, int num_kv_heads, int head_dim,
                    int block_size, int64_t num_blocks, float softmax_scale,
                    int num_splits, int split_tokens,
                    void *workspace, int64_t workspace_bytes,
                    int q_dtype, int kv_dtype,
                    const float *k_scale, const float *v_scale, void *stream);

/*
 * nq_paged_decode with Qwen3.5's attention output gate applied in the output
 * store.  Replaces the decode call (layers/attention.py:72-74) together with
 * the gating that follows it in Qwen3_5Attention.forward
 * (models/qwen3_5.py:140-142):  out = rnd(rnd(o) * rnd(sigmoid(gate))),
 * sigmoid(g) = 1 / (1 + exp(-g)) in fp32, rnd = round to the q/out type --
 * eager torch's arithmetic for 16-bit tensors.
 * gate [batch, num_q_heads, head_dim] has the type of q/out, strides
 * (gate_batch_stride, gate_head_stride, 1), 8-byte aligned (for example the
 * gate half of q_proj's [B, Hq, 2*D] output).  Rows with context_len <= 0
 * stay zero.  Every other argument is as for nq_paged_decode.
 */
int nq_paged_decode_gated(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                          const void *k_cache, const void *v_cache,
                          const int32_t *block_tables, int64_t bt_stride,
                          int max_blocks_per_seq, const int32_t *context_lens,
                          void *out, int64_t out_batch_stride, int64_t out_head_stride,
                          int batch, int num_q_heads, int num_kv_heads, int head_dim,
                          int block_size, int64_t num_blocks, float softmax_scale,
                          int num_splits, int split_tokens,
                          void *workspace, int64_t workspace_bytes,
                          int q_dtype, int kv_dtype,
                          const float *k_scale, const float *v_scale,
                          const void *gate, int64_t gate_batch_stride, int64_t gate_head_stride,
                          void *stream);

/*
 * The decode step of Attention.forward in one launch: the new token's KV
 * store and the paged decode.  Replaces store_kvcache(k, v, k_cache, v_cache,
 * slot_mapping) followed by flash_attn_with_kvcache(...)
 * (layers/attention.py:62-63 then :71-74); with a non-NULL gate, also the
 * gating of models/qwen3_5.py:140-142 (as nq_paged_decode_gated).
 *
 * k_new / v_new [batch, num_kv_heads, head_dim] with row strides
 * k_new_row_stride / v_new_row_stride (elements of new_dtype), 16-byte
 * aligned rows contiguous over (head, dim); new_dtype == kv_dtype for a
 * 16-bit cache, or F32/F16/BF16 for an fp8 cache (quantized with
 * k_scale/v_scale exactly as nq_store_kvcache does).  slot_mapping [batch]
 * int32: row b goes to cache row slot_mapping[b] when that lies in
 * [0, num_blocks * block_size) (-1 skips it).  Every other argument is as
 * for nq_paged_decode / nq_paged_decode_gated; gate may be NULL.
 *
 * Cache bytes and outputs equal those of nq_store_kvcache followed by
 * nq_paged_decode(_gated) when, for every sequence b, slot_mapping[b] is -1
 * or the slot of token context_lens[b] - 1 in b's block table (what
 * engine/decode_init.py writes) and no other sequence of the batch reads
 * that slot.  The workgroup that reads that token takes it from k_new/v_new
 * instead of the cache, so the store and the attention need no ordering.
 */
int nq_paged_decode_store(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                          void *k_cache, void *v_cache,
                          const int32_t *block_tables, int64_t bt_stride,
                          int max_blocks_per_seq, const int32_t *context_lens,
                          const void *k_new, int64_t k_new_row_stride,
                          const void *v_new, int64_t v_new_row_stride,
                          const int32_t *slot_mapping, int new_dtype,
                          void *out, int64_t out_batch_stride, int64_t out_head_stride,
                          int batch, int num_q_heads, int num_kv_heads, int head_dim,
                          int block_size, int64_t num_blocks, float softmax_scale,
                          int num_splits, int split_tokens,
                          void *workspace, int64_t workspace_bytes,
                          int q_dtype, int kv_dtype,
                          const float *k_scale, const float *v_scale,
                          const void *gate, int64_t gate_batch_stride, int64_t gate_head_stride,
                          void *stream);

/*
 * nq_paged_decode without a caller workspace, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference: it is
 * nq_paged_decode with the split-K partials in a static device array of
 * NQ_DECODE_NOALLOC_SCRATCH_BYTES per device, which each device holds until
 * the process ends.  It calls no allocating routine; the array's address is
 * looked up (hipGetSymbolAddress) on the first call on each device.
 * Every other argument is as for nq_paged_decode.  A plan whose splits
 * were grown past the table (nq_decode_plan sizes a stream-K workspace that
 * way) runs with the splits that cover the table when the grown plan's
 * nq_decode_workspace_bytes exceeds the array; only a plan whose covering
 * splits still need more than the array returns NQ_EINVAL.  All calls on one
 * device share its array, which keeps the last call's partials: calls that
 * overlap on one device (several streams or host threads) race and must be
 * ordered by the caller.  Loading the library reserves the array on every
 * device it runs on (64 MiB of HBM each) until the process ends.
 */
#define NQ_DECODE_NOALLOC_SCRATCH_BYTES (64LL << 20)
int nq_paged_decode_noalloc(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                            const void *k_cache, const void *v_cache,
                            const int32_t *block_tables, int64_t bt_stride,
                            int max_blocks_per_seq, const int32_t *context_lens,
                            void *out, int64_t out_batch_stride, int64_t out_head_stride,
                            int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int block_size, int64_t num_blocks, float softmax_scale,
                            int num_splits, int split_tokens,
                            int q_dtype, int kv_dtype,
                            const float *k_scale, const float *v_scale, void *stream);

/*
 * Qwen3.5's attention output gate as one in-place pass:
 *   out[i, h, :] = rnd(out[i, h, :] * rnd(sigmoid(gate[i, h, :])))
 * Replaces attn_output * torch.sigmoid(gate) (models/qwen3_5.py:140-142)
 * after the prefill call.  out and gate are [num_tokens, num_heads,
 * head_dim] of type dtype (F16/BF16) with (row, head) strides; every pointer
 * and stride 16-byte aligned; head_dim a multiple of 8.
 */
int nq_output_gate(void *out, int64_t out_row_stride, int64_t out_head_stride,
                   const void *gate, int64_t gate_row_stride, int64_t gate_head_stride,
                   int64_t num_tokens, int num_heads, int head_dim, int dtype, void *stream);

/*
 * Causal varlen prefill attention, optionally over paged K/V.
 * Replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q=..., cu_seqlens_k=...,
 *   max_seqlen_q=..., max_seqlen_k=..., softmax_scale=scale, causal=True,
 *   block_table=block_tables)   (layers/attention.py:64-70).
 *
 * head_dim is 128 or 256 (NQ_EUNSUPPORTED otherwise).
 * q [total_q, num_q_heads, head_dim] (strides q_row_stride, q_head_stride, 1),
 * out likewise.  Sequence s owns query rows [cu_q[s], cu_q[s+1]) and
 * Lk = cu_k[s+1]-cu_k[s] keys; query row i (0-based in s) sees keys
 * j <= i + Lk - Lq (bottom-right causal) when causal != 0, all Lk keys
 * otherwise.
 * block_tables == NULL: k/v are packed [total_k, num_kv_heads, head_dim]
 *   with row stride kv_row_stride; key j of s is row cu_k[s] + j.
 * block_tables != NULL: k/v are the paged caches; key j of s is cache row
 *   block_tables[s*bt_stride + j/block_size]*block_size + j%block_size.
 * kv_dtype == q_dtype (F16/BF16), or NQ_FP8_E4M3 with k_scale/v_scale.
 * q, k, v and out (base pointers, row and head strides) must be 16-byte
 * aligned (NQ_EINVAL otherwise); a K/V row stride is at most 1 MiB.
 * workspace:>= nq_prefill_workspace_bytes() bytes, 4-byte aligned, all zero
 * before its first use; every completed call leaves it zero again, so it is
 * allocated and cleared once and then reused (also under graph replay).
 * Calls that share a workspace must not run concurrently.
 */
int nq_varlen_prefill(const void *q, int64_t q_row_stride, int64_t q_head_stride,
                      const void *k, const void *v, int64_t kv_row_stride,
                      const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                      int max_seqlen_q, int max_seqlen_k,
                      const int32_t *block_tables, int64_t bt_stride,
                      int max_blocks_per_seq, int64_t num_blocks,
                      void *out, int64_t out_row_stride, int64_t out_head_stride,
                      int num_seqs, int num_q_heads, int num_kv_heads,
                      int head_dim, int block_size, float softmax_scale,
                      int causal, int q_dtype, int kv_dtype,
                      const float *k_scale, const float *v_scale,
                      void *workspace, int64_t workspace_bytes, void *stream);

/*
 * nq_varlen_prefill with Qwen3.5's attention output gate (models/qwen3_5.py:
 * 140-142): out = rnd(rnd(o) * rnd(sigmoid(gate))) as for
 * nq_paged_decode_gated.  gate [total_q, num_q_heads, head_dim] has the type
 * of q/out, strides (gate_row_stride, gate_head_stride, 1), 16-byte aligned
 * (e.g. the gate half of q_proj's output); total_q = cu_seqlens_q[num_seqs].
 * The kernels apply the gate in their own output stores (a non-default
 * launch shape, NQ_PREFILL_SHAPE=a, is followed by one nq_output_gate pass on
 * the same stream instead).
 */
int nq_varlen_prefill_gated(const void *q, int64_t q_row_stride, int64_t q_head_stride,
                            const void *k, const void *v, int64_t kv_row_stride,
                            const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                            int max_seqlen_q, int max_seqlen_k,
                            const int32_t *block_tables, int64_t bt_stride,
                            int max_blocks_per_seq, int64_t num_blocks,
                            void *out, int64_t out_row_stride, int64_t out_head_stride,
                            int num_seqs, int num_q_heads, int num_kv_heads,
                            int head_dim, int block_size, float softmax_scale,
                            int causal, int q_dtype, int kv_dtype,
                            const float *k_scale, const float *v_scale,
                            void *workspace, int64_t workspace_bytes,
                            const void *gate, int64_t gate_row_stride, int64_t gate_head_stride,
                            int64_t total_q, void *stream);

/* Bytes of device workspace nq_varlen_prefill needs (work-queue counters). */
int64_t nq_prefill_workspace_bytes(void);

/*
 * Decode metadata on the device.
 * Replaces _prepare_decode_kernel (engine/decode_init.py:6-65):
 *   input_ids[i]    = sampled_token_ids[batch_slots[i]]
 *   positions[i]    = seq_lens[i] - 1
 *   context_lens[i] = seq_lens[i]
 *   slot_mapping[i] = last_block_ids[i]*block_size + (seq_lens[i]-1) % block_size
 * for i < num_seqs.
 */
int nq_prepare_decode(const int64_t *sampled_token_ids, const int64_t *batch_slots,
                      const int32_t *seq_lens, const int32_t *last_block_ids,
                      int64_t *input_ids, int64_t *positions,
                      int32_t *context_lens, int32_t *slot_mapping,
                      int num_seqs, int block_size, void *stream);

/*
 * Fused q/k Gemma RMS norm + partial rotary embedding + KV-cache store.
 * Replaces, in Qwen3_5Attention.forward (models/qwen3_5.py:135-137), the
 * calls q_norm(query), k_norm(key) (GemmaRMSNorm, layers/layernorm.py:81-91)
 * and rotary_emb(positions, query, key) (InterleavedMRoPE,
 * layers/rotary_embedding.py:104-123), plus the store that Attention.forward
 * then makes (layers/attention.py:62-63).
 *
 * q [num_tokens, num_q_heads, head_dim] with strides (q_row_stride,
 * q_head_stride, 1) -- e.g. the query half of q_proj's [N, Hq, 2*D] output;
 * k and v [num_tokens, num_kv_heads, head_dim] with row strides and head
 * stride head_dim.  dtype (F32/F16/BF16) is the type of q, k, v, both
 * weights [head_dim] and both outputs.  For each row x of a head:
 *   y = rnd(rnd(x / sqrt(mean(x^2) + eps)) * (w + weight_offset))
 * (fp32 arithmetic, rnd = round to dtype; weight_offset is 1.0 for the
 * Gemma norm), then the first rotary_dim dims rotate by the table row
 * cos_sin_cache[positions[i]] (float32 [max_position, rotary_dim]: the
 * rotary_dim/2 cosines, then the sines):
 *   e <  R/2: z[e] = rnd(y[e]*cos[e] - y[e+R/2]*sin[e])
 *   e >= R/2: z[e] = rnd(y[e]*cos[e-R/2] + y[e-R/2]*sin[e-R/2])
 * rotary_dim is a multiple of 16 in [0, head_dim]; head_dim is 64, 128 or
 * 256; positions are int64, and a position outside [0, max_position) gives a
 * NaN row.  q_out (strides q_out_row_stride, q_out_head_stride, 1) receives
 * the rotated q; k_out (row stride k_out_row_stride, may be NULL) the rotated
 * k.  Outputs may alias their inputs with equal strides (in place).
 * k_cache/v_cache == NULL: no store (the reference skips it while the caches
 * are empty).  Otherwise the rotated k row and the v row of token i go to
 * cache row slot_mapping[i] exactly as nq_store_kvcache stores them
 * (cache_dtype == dtype, or NQ_FP8_E4M3 with k_scale/v_scale); slots outside
 * [0, num_slots) are skipped.  Every pointer and stride must be 16-byte
 * aligned.
 */
int nq_qk_norm_rope_store(const void *q, int64_t q_row_stride, int64_t q_head_stride,
                          const void *k, int64_t k_row_stride,
                          const void *v, int64_t v_row_stride,
                          const int64_t *positions, const float *cos_sin_cache,
                          int64_t max_position, int rotary_dim,
                          const void *q_weight, const void *k_weight,
                          float eps, float weight_offset,
                          void *q_out, int64_t q_out_row_stride, int64_t q_out_head_stride,
                          void *k_out, int64_t k_out_row_stride,
                          void *k_cache, void *v_cache, const int32_t *slot_mapping,
                          int64_t num_slots, int64_t num_tokens,
                          int num_q_heads, int num_kv_heads, int head_dim,
                          int dtype, int cache_dtype,
                          const float *k_scale, const float *v_scale, void *stream);

/*
 * Gated DeltaNet decode step for a whole batch, on a pool of recurrent
 * states updated in place.  Replaces decode_gated_delta_rule
 * (layers/gated_delta_net.py:85-122, FlashInfer's
 * gated_delta_rule_decode_pretranspose with use_qk_l2norm=True, called once
 * per sequence by models/qwen3_5.py:226-240) together with the state slot's
 * read and write around it (layers/gated_delta_net.py:168-173, 250-262).
 *
 * For sequence b < batch with slot = state_indices[b] in [0, num_slots)
 * (other slots: the sequence is skipped, out untouched) and value head hv
 * (key head h = hv / (num_v_heads / num_k_heads)), S = state[slot, hv]
 * ([head_v_dim, head_k_dim] fp32, K-last), in fp32:
 *   q, k = x / sqrt(sum(x^2) + 1e-6) of q[b, h], k[b, h]
 *   g    = -exp(A_log[hv]) * softplus(a[b, hv] + dt_bias[hv])
 *          (softplus(x) = x for x > 20, else log1p(exp(x)))
 *   beta = sigmoid(b[b, hv])
 *   S    = exp(g) * S;  u = beta * (v[b, hv] - S k);  S = S + u k^T
 *   out[b, hv] = S q / sqrt(head_k_dim)       (rounded to dtype)
 * q, k [batch, num_k_heads, 128] and v, out [batch, num_v_heads, 128] are
 * contiguous over (head, dim) with the given row strides; a, b [batch,
 * num_v_heads]; all of type dtype (F16/BF16).  A_log, dt_bias float
 * [num_v_heads]; state float [num_slots, num_v_heads, 128, 128], 16-byte
 * aligned; q and k rows 8-byte aligned.  head_k_dim = head_v_dim = 128 (NQ_EUNSUPPORTED otherwise).
 * Sequences of one call must use distinct slots.
 */
int nq_gdn_decode(const void *q, int64_t q_row_stride, const void *k, int64_t k_row_stride,
                  const void *v, int64_t v_row_stride, const void *a, int64_t a_row_stride,
                  const void *b, int64_t b_row_stride, const float *A_log, const float *dt_bias,
                  float *state, const int32_t *state_indices, int64_t num_slots,
                  void *out, int64_t out_row_stride, int batch, int num_k_heads, int num_v_heads,
                  int head_k_dim, int head_v_dim, int dtype, void *stream);

/*
 * Gated DeltaNet prefill for a batch of sequences, in the chunked (WY) form
 * over 64-token chunks on MFMA.
 * Replaces chunk_gated_delta_rule (layers/gated_delta_net.py:44-82, the
 * Triton chunk kernels of layers/fla/ with use_qk_l2norm_in_kernel=True and
 * initial_state=None), the gating computed before it (:197-198) and the
 * final-state write to the pool after it (:210-214), called per sequence by
 * models/qwen3_5.py:215-224.
 * Sequence n < num_seqs owns token rows [cu_seqlens[n], cu_seqlens[n+1]) of
 * q, k [T, num_k_heads, 128], v, out [T, num_v_heads, 128] and a, b
 * [T, num_v_heads].  Its state starts at zero (initial_state_from_slot == 0,
 * as in the reference) or at state[state_indices[n]], follows the step of
 * nq_gdn_decode over the tokens in order, writing out for every token, and
 * is stored to state[state_indices[n]] (a slot outside [0, num_slots) keeps
 * nothing and starts from zero).  Products take 16-bit operands with
 * float32 accumulation, as the reference's kernels do; the state stays
 * float32 between chunks.  Types as for nq_gdn_decode; q, k, v, out and
 * their row strides 16-byte aligned; cu_seqlens int32 [num_seqs + 1].
 * out is also the kernel's scratch: the first 16 bytes of each (token, value
 * head) row hold that token's gate values until its output is written, so
 * out must not overlap q, k, v, a or b.
 */
int nq_gdn_prefill(const void *q, int64_t q_row_stride, const void *k, int64_t k_row_stride,
                   const void *v, int64_t v_row_stride, const void *a, int64_t a_row_stride,
                   const void *b, int64_t b_row_stride, const float *A_log, const float *dt_bias,
                   const int32_t *cu_seqlens, int num_seqs, float *state,
                   const int32_t *state_indices, int64_t num_slots, int initial_state_from_slot,
                   void *out, int64_t out_row_stride, int num_k_heads, int num_v_heads,
                   int head_k_dim, int head_v_dim, int dtype, void *stream);

/*
 * Gated RMS norm of the Gated DeltaNet output, one pass.
 * Replaces RMSNormGated.forward (layers/layernorm.py:143-157) as applied by
 * GatedDeltaNet (self.norm(out, z), layers/gated_delta_net.py:205-207,
 * 268-270).  For each of `rows` rows of dim elements (x and gate of type
 * dtype, F16/BF16; weight float [dim]), in fp32, rnd = round to dtype:
 *   n = rnd(x / sqrt(mean(x^2) + eps))
 *   out = rnd(rnd(n * rnd(weight)) * gate / (1 + exp(-gate)))
 * dim is 64, 128 or 256; pointers and row strides 16-byte aligned; out may
 * alias x.
 */
int nq_gated_rmsnorm(const void *x, int64_t x_row_stride, const void *gate, int64_t gate_row_stride,
                     const float *weight, float eps, void *out, int64_t out_row_stride,
                     int64_t rows, int dim, int dtype, void *stream);

/*
 * Causal depthwise conv1d + silu in front of the Gated DeltaNet, with the
 * conv state pool.  Replaces, in GatedDeltaNet (layers/gated_delta_net.py),
 * silu(conv1d(qkv)[:, :, :S]) and the state kept for decode (prefill,
 * :178-180, 207-213) and x = cat(conv_state, qkv); silu(conv1d(x)); the new
 * state x[:, 1:] (decode, :218-227).
 * x, out [rows, channels] (16-bit dtype; row strides, in elements, at least
 * channels: NQ_EINVAL otherwise), weight [channels, kernel_size]
 * (dtype; the reference's conv1d.weight [C, 1, K]), conv_state
 * [num_slots, channels, kernel_size - 1] (dtype, oldest input first).
 * cu_seqlens == NULL (decode): sequence b is row b, its window is the slot's
 *   state then x[b]; the slot then holds the last K - 1 inputs.
 * cu_seqlens != NULL (prefill): sequence n owns rows [cu[n], cu[n+1]), its
 *   window starts from zeros (initial_state_from_slot must be 0, as in the
 *   reference); its slot receives its last K - 1 inputs.
 * out = rnd(y / (1 + exp(-y))), y = rnd(sum_j w[c][j] x[t-K+1+j]) in fp32.
 * Slots outside [0, num_slots) skip the state.  kernel_size in [2, 8].
 */
int nq_gdn_conv1d(const void *x, int64_t x_row_stride, const void *weight, int kernel_size,
                  const int32_t *cu_seqlens, int num_seqs, void *conv_state,
                  const int32_t *state_indices, int64_t num_slots, int initial_state_from_slot,
                  void *out, int64_t out_row_stride, int channels, int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NQ_ATTN_H */
