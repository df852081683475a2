/* Decode-step operators around the quantized linears (batch-1 Qwen3 decode).
 *
 * These are the callers on either side of the quantized Linear in the
 * reference's Qwen3 decoder layer (ondeviceinfer/quantized_model.py:124-228):
 * residual add + RMSNorm, SiLU(gate) * up, and single-token grouped-query
 * attention over a resident fp16 KV cache with Qwen3's per-head q/k RMSNorm,
 * rotary embedding and the cache append folded into one launch.
 *
 * Same conventions as ondeviceinfer_wq.h: device pointers, fp16 as uint16_t,
 * `stream` is a hipStream_t (may be NULL), 0 or a WQ_ERR_* code is returned and
 * wq_last_error() holds the message, nothing allocates or synchronizes, and
 * every call may be captured in a HIP graph.
 */
#ifndef ONDEVICEINFER_DECODE_H
#define ONDEVICEINFER_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out_sum[r] = x[r] + delta[r] (fp16 add; delta may be NULL, then x itself);
 * out_norm[r] = weight * fp16(out_sum[r] * rsqrt(mean(out_sum[r]^2) + eps)),
 * the reduction in fp32, for rows r < rows of n elements (n % 8 == 0).
 * out_sum may be NULL (not written) or alias x.
 * Replaces: `residual + attention_output` (quantized_model.py:211) followed
 * by rms_norm (functional.py:17-22; called at quantized_model.py:147, :214). */
int wq_add_rmsnorm(const uint16_t* x, const uint16_t* delta, const uint16_t* weight, int64_t rows, int64_t n,
                   float eps, uint16_t* out_norm, uint16_t* out_sum, void* stream);

/* out[r, i] = fp16(fp16(silu(gate_up[r, i])) * gate_up[r, n + i]) for the
 * concatenated [gate | up] rows of a fused gate_up projection (n % 8 == 0).
 * Replaces: `F.silu(gate) * up` (quantized_model.py:222-224). */
int wq_silu_mul(const uint16_t* gate_up, int64_t rows, int64_t n, uint16_t* out, void* stream);

/* Workspace bytes for wq_decode_attention at this geometry (0 when one
 * workgroup covers each kv head's cache).  The workspace holds the chunk
 * partials between the attention launch and its merge launch; it needs no
 * initialization, and calls that may overlap need separate workspaces. */
int wq_decode_attention_workspace_size(int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq,
                                       size_t* bytes);

/* One decode token of Qwen3 self-attention, batch 1, head_dim 128.
 *   qkv          [q_heads*128 | kv_heads*128 | kv_heads*128] projection output
 *   q/k_norm     per-head RMSNorm weights [128] (NULL: no norm)
 *   cos/sin      RoPE tables [>= max_seq, 128] fp16, row p for position p
 *   position     device int32: the token's position p; keys 0..p are attended
 *   key/value_cache [kv_heads, max_seq, 128] fp16; row p is written here
 *   out          [q_heads*128] attention output (before o_proj)
 * Replaces: q/k rms_norm + apply_rotary_pos_emb + ResidentKVCache.update +
 * F.scaled_dot_product_attention(enable_gqa=True) for query_length 1
 * (quantized_model.py:171-199, layers.py:64-80, cache.py:60-80,
 * attention.py:35-85).  max_seq <= 16384, q_heads / kv_heads <= 8.  A
 * position outside [0, max_seq) writes NaN to out and leaves the cache
 * untouched. */
int wq_decode_attention(const uint16_t* qkv, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                        const uint16_t* q_norm_weight, const uint16_t* k_norm_weight, float eps,
                        const uint16_t* cos_table, const uint16_t* sin_table, const int32_t* position,
                        uint16_t* key_cache, uint16_t* value_cache, int64_t max_seq, float scale, uint16_t* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Prefill (tokens >= 1, batch 1) q/k RMSNorm + RoPE with the cache append:
 *   qkv          [tokens, q_heads*128 | kv_heads*128 | kv_heads*128] fused
 *                projection output, row t at position start + t
 *   q/k_norm     per-head RMSNorm weights [128] (NULL: no norm)
 *   cos/sin_rows [tokens, 128] fp16 RoPE rows of those positions
 *   key/value_cache [kv_heads, max_seq, 128] fp16; rows start .. start+tokens-1
 *                receive the normalized, rotated k and the v
 *   q_out        [tokens, q_heads, 128] normalized, rotated q (token-major,
 *                the layout a fused attention reads as [q_heads, tokens, 128]
 *                strided and writes its output in)
 * Same numerics per element as wq_decode_attention's prologue.  Replaces:
 * the q/k rms_norm + apply_rotary_pos_emb of a multi-token forward
 * (quantized_model.py:177-184, layers.py:64-80) and the cache.update inside
 * its cached attention (quantized_model.py:186-195, attention.py:35-85,
 * cache.py:60-80).  start + tokens <= max_seq. */
int wq_prefill_qk_rope(const uint16_t* qkv, int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                       const uint16_t* q_norm_weight, const uint16_t* k_norm_weight, float eps,
                       const uint16_t* cos_rows, const uint16_t* sin_rows, int64_t start, uint16_t* key_cache,
                       uint16_t* value_cache, int64_t max_seq, uint16_t* q_out, void* stream);

/* Prefill (tokens >= 1, batch 1) causal grouped-query attention over the
 * resident cache, head_dim 128:
 *   q            [tokens, q_heads, 128] fp16, token-major (wq_prefill_qk_rope's
 *                q_out), query t at position start + t
 *   key/value_cache [kv_heads, max_seq, 128] fp16; rows 0 .. start+tokens-1
 *                hold the keys and values (this call's rows appended already)
 *   out          [tokens, q_heads, 128] fp16, token-major
 * Query t attends keys 0 .. start + t with weights softmax(scale * q.k),
 * accumulated in fp32 with the probabilities rounded to fp16 for the value
 * product (flash-attention order: the scores never reach memory).
 * Replaces: F.scaled_dot_product_attention(is_causal / absolute causal mask,
 * enable_gqa=True) over the cached keys in a multi-token forward
 * (attention.py:35-85, quantized_model.py:186-199). */
int wq_prefill_attention(const uint16_t* q, int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                         const uint16_t* key_cache, const uint16_t* value_cache, int64_t max_seq, int64_t start,
                         float scale, uint16_t* out, void* stream);

/* Workspace bytes for wq_lm_head with token != NULL (the per-wave argmax
 * candidates; no initialization needed). */
int wq_lm_head_workspace_size(int64_t k, int64_t vocab, size_t* bytes);

/* The fp16 LM head of one decode token and its greedy token:
 *   logits[v] = fp16(sum_k weight[v, k] * x[k])  (fp32 accumulation), and
 *   *token    = the first v with the largest logits[v] (NaN counts as the
 *               largest value), i.e. torch.argmax over the fp16 logits.
 * weight is the row-major fp16 [vocab, k] LM-head matrix, k % 512 == 0 and
 * k <= 8192; logits (fp16 [vocab]) or token (one int64) may be NULL, not
 * both.  x and weight 16-byte aligned.
 * Replaces: `F.linear(hidden_states, self.lm_head)` (quantized_model.py:337)
 * and `output.logits[:, -1].argmax(dim=-1, keepdim=True)` (generation.py:47,
 * :58) for one token. */
int wq_lm_head(const uint16_t* x, int64_t k, const uint16_t* weight, int64_t vocab, uint16_t* logits,
               int64_t* token, void* workspace, size_t workspace_bytes, void* stream);

/* wq_lm_head on the model's final RMSNorm of x, formed inside the LM head
 * kernel: x is the final residual stream [k] and the LM head reads
 * norm_weight * fp16(x * rsqrt(sum(sumsq_in) / k + eps)) (fp32 normalize,
 * fp16 cast, fp16 scale), where sumsq_in holds the sums of squares of x over
 * 16-element tiles (0 < sumsq_count <= 1024), as the fused decode linears'
 * residual epilogue writes them.  norm_weight 16-byte aligned.
 * Replaces: `rms_norm(hidden_states, self.final_norm, eps)` followed by the
 * LM head and the greedy token (quantized_model.py:331-337, functional.py:17-22,
 * generation.py:47, :58) for one decode token, without the norm's launch. */
int wq_lm_head_rmsnorm(const uint16_t* x, int64_t k, const uint16_t* norm_weight, const float* sumsq_in,
                       int64_t sumsq_count, float eps, const uint16_t* weight, int64_t vocab, uint16_t* logits,
                       int64_t* token, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for wq_argmax_f16 (per-wave candidates; no initialization
 * needed). */
int wq_argmax_f16_workspace_size(int64_t n, size_t* bytes);

/* *token = the first index of the largest of n fp16 values (NaN counts as the
 * largest), i.e. torch.argmax over a 1-D fp16 tensor; 1 <= n <= 2^30, x
 * 16-byte aligned.  For logits that another kernel produced (the W4 LM head
 * of a decode step).  Replaces `output.logits[:, -1].argmax(dim=-1,
 * keepdim=True)` (generation.py:47, :58) for one token. */
int wq_argmax_f16(const uint16_t* x, int64_t n, int64_t* token, void* workspace, size_t workspace_bytes,
                  void* stream);

/* *device_ptr = the address kernels use for pinned host memory at host_ptr
 * (hipHostGetDevicePointer); WQ_ERR_INVALID_ARGUMENT when host_ptr is not in
 * a device-mapped pinned allocation.  Not a stream operation.  Used to hand
 * wq_embed_rows the embedding table that stays in host memory, as the
 * reference keeps it (quantized_model.py:289-291). */
int wq_host_device_pointer(const void* host_ptr, void** device_ptr);

/* out[r, :] = table[tokens[r], :] for r < rows: the embedding rows of fp16
 * [vocab, hidden] (hidden % 8 == 0) for device int64 token ids; table may be
 * the device address of pinned host memory (wq_host_device_pointer), read over
 * the host link.  A token outside [0, vocab) writes NaN and reads nothing.
 * sumsq_out (may be NULL; hidden % 16 == 0) receives, per row, the fp32 sum of
 * squares of each 16 consecutive elements ([rows, hidden / 16]): what the
 * fused decode linears' RMSNorm prologue takes (the first layer's input norm).
 * table and out 16-byte aligned.
 * Replaces: `F.embedding(ids_cpu, self.store.embed_tokens)` + `.to(device)`
 * (quantized_model.py:289-291) for a token id that is already on the device
 * (the previous decode step's greedy token). */
int wq_embed_rows(const uint16_t* table, int64_t vocab, int64_t hidden, const int64_t* tokens, int64_t rows,
                  uint16_t* out, float* sumsq_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ONDEVICEINFER_DECODE_H */
