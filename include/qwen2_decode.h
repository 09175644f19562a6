/*
 * qwen2_decode.h -- C ABI of the fused decode-step kernels that sit between
 * the W4G64 linears of a Qwen2 decoder layer (one token per sequence, bf16
 * hidden states).  Same conventions as w4g64.h: plain device pointers, sizes,
 * a HIP stream as `void*`, int status codes W4G64_STATUS_*, the message of a
 * failed call in w4g64_last_error().  Nothing here allocates or synchronizes.
 *
 * With these, one decoder layer's decode step is at most seven launches:
 *   add_rmsnorm -> W4G64 q|k|v (one N = (H + 2 KVH) * D launch, bias)
 *   -> decode_attention -> W4G64 o_proj -> add_rmsnorm
 *   -> W4G64 gate|up (one N = 2 I launch) -> W4G64 down_proj,
 * and the step ends with add_rmsnorm -> lm_head (logits and greedy token).
 * At batch 1 it is five: each add_rmsnorm after the first is formed in the
 * staging of the linear that follows it (w4g64_linear_rmsnorm), and the down
 * projection's K-split partial sums are added there too
 * (w4g64_linear_partials, W4G64_DTYPE_F32_PARTIALS).
 */
#ifndef QWEN_INT4_HIP_QWEN2_DECODE_H
#define QWEN_INT4_HIP_QWEN2_DECODE_H

#include <stdint.h>

#include "w4g64.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Start of a decode step for `batch` sequences at the common position
 * p = *position (a device int64):
 *   x[b]   = embed[token_ids[b]]               (bf16 [batch, hidden]; a row of NaN
 *                                                for an id outside [0, vocab))
 *   cos[b][d], sin[b][d] = bf16(cos / sin(float(p) * inv_freq[d % (head_dim / 2)]))
 *                                              (bf16 [batch, head_dim], fp32 math)
 *   normed[b] = bf16(bf16(x[b] * rsqrt(mean(x[b]^2) + eps)) * norm_weight)
 *                                              (only when norm_weight and normed are
 *                                                given: the first layer's input norm)
 * token_ids int64 [batch], embed bf16 [vocab, hidden] (16-byte aligned, as x,
 * norm_weight and normed), inv_freq fp32 [head_dim / 2] (the rotary module's
 * buffer).  head_dim == 128.
 * Replaces: the embedding lookup of QwenModel.forward, RotaryEmbedding.forward
 *           for one position and the first layer's input RMSNorm
 *           (src/qwen_int4/model.py:22-31, :40-44, :182, :190). */
int qwen2_decode_prologue(const int64_t* token_ids, const void* embed, const int64_t* position, const float* inv_freq,
                          void* x, void* cos, void* sin, const void* norm_weight, float eps, void* normed,
                          int64_t batch, int64_t hidden, int64_t vocab, int64_t head_dim, void* stream);

/* Residual add + RMSNorm over `rows` rows of `hidden` bf16 values:
 *   s        = x                                   (delta == NULL)
 *            = bf16(x + bf16(delta))               (delta bf16, fp32, or fp32 partial
 *                                                   sums: W4G64_DTYPE_F32_PARTIALS)
 *   out_sum  = s                                   (may be NULL; may alias x)
 *   out_norm = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * weight)
 * in fp32 arithmetic with the reference's two roundings.  hidden is a
 * multiple of 8, at most 8192; all pointers 16-byte aligned.
 * Replaces: RMSNorm.forward (src/qwen_int4/model.py:40-44) and the residual
 *           adds of DecoderLayer.forward (model.py:149-154; the MLP output is
 *           cast to bf16 first, model.py:136). */
int qwen2_add_rmsnorm(const void* x, const void* delta, int delta_dtype, const void* weight, float eps,
                      void* out_sum, void* out_norm, int64_t rows, int64_t hidden, void* stream);

/* Bytes of workspace qwen2_decode_attention needs (arrival counters, then
 * fp32 per-chunk partial results).  The counter area must be zero before the
 * first call; every call leaves it zero.  Calls sharing a workspace must be
 * ordered on one stream. */
int64_t qwen2_decode_attention_workspace_bytes(int64_t batch, int64_t num_kv_heads, int64_t max_length);

/* One decode step of grouped-query attention for `batch` sequences that all
 * sit at the same position p = *position (a device int64; clamped to
 * [0, max_length)):
 *   qkv      bf16 [batch, (num_heads + 2 num_kv_heads) * head_dim]: the fused
 *            q|k|v projection of the new token (bias included);
 *   cos, sin bf16 [batch, head_dim]: the rotary factors of position p;
 *   k_cache, v_cache bf16 [batch, num_kv_heads, max_length, head_dim].
 * Rotates q and k as q * cos + rotate_half(q) * sin with bf16 rounding after
 * each product and after the sum, writes the rotated key and the value at
 * position p, and writes
 *   out[b, h * head_dim + d] = bf16( softmax_t(q_h . k_t * scale) . v_t[d] ),
 *   t = 0..p, query head h reading key/value head h / (num_heads / num_kv_heads),
 * with fp32 scores, softmax and sums.  head_dim == 128,
 * num_heads / num_kv_heads <= 8, max_length <= 17408.  qkv, the caches and
 * the workspace must be 16-byte aligned, out 8-byte aligned.
 * Replaces: the rotary step and attention of QwenAttention.forward for one
 *           cached token (src/qwen_int4/model.py:17-31, :61-122). */
int qwen2_decode_attention(const void* qkv, const void* cos, const void* sin, void* k_cache, void* v_cache,
                           const int64_t* position, void* out, int64_t batch, int64_t num_heads,
                           int64_t num_kv_heads, int64_t head_dim, int64_t max_length, float scale,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* qwen2_decode_attention without its merge: the same rotary step and cache
 * write, and every 64-position chunk's workgroup leaves its partial result
 * (per query head: score maximum m_c, sum l_c of exp(score - m_c), and the
 * exp-weighted value sums acc_c[128], fp32) in the workspace; chunks past the
 * position leave m_c = -inf, l_c = 0 and zero sums.  No output row is
 * written: w4g64_linear_attention_merge merges the chunks in the staging of
 * the o_proj linear, with the result qwen2_decode_attention would have
 * written.  Same arguments and workspace as qwen2_decode_attention, minus
 * `out`; the counter area is left untouched.
 * Replaces: with w4g64_linear_attention_merge, the rotary step, attention and
 *           o_proj of QwenAttention.forward for one cached token
 *           (src/qwen_int4/model.py:17-31, :61-122). */
int qwen2_decode_attention_partials(const void* qkv, const void* cos, const void* sin, void* k_cache,
                                    void* v_cache, const int64_t* position, int64_t batch, int64_t num_heads,
                                    int64_t num_kv_heads, int64_t head_dim, int64_t max_length, float scale,
                                    void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of workspace qwen2_prefill_attention needs: the rotated queries,
 * bf16 [batch, num_heads, length, head_dim]. */
int64_t qwen2_prefill_attention_workspace_bytes(int64_t batch, int64_t num_heads, int64_t length);

/* Attention over a prompt of `length` positions per sequence.
 *   qkv bf16 [batch * length, (num_heads + 2 num_kv_heads) * head_dim] (q | k | v
 *     projections of every position, row b * length + i);
 *   cos, sin bf16 [batch * length, head_dim]: the rotary factors of position i;
 *   k_cache, v_cache bf16 [batch, num_kv_heads, max_length, head_dim].
 * Rotates q and k as qwen2_decode_attention does, writes the rotated keys and
 * the values at positions 0..length-1 of the caches (later positions are left
 * alone), and writes
 *   out[b * length + i, h * head_dim + d] =
 *       bf16( softmax_{t <= i}(q_{h,i} . k_t * scale) . v_t[d] )
 * with fp32 scores, softmax and sums (causal mask).  head_dim == 128,
 * num_heads / num_kv_heads <= 8, length <= max_length; qkv, the caches and
 * the workspace 16-byte aligned.
 * Replaces: the rotary step, cache update and attention of
 *           QwenAttention.forward over a prompt (src/qwen_int4/model.py:17-31,
 *           :61-122, the causal mask of :94-120). */
int qwen2_prefill_attention(const void* qkv, const void* cos, const void* sin, void* k_cache, void* v_cache,
                            void* out, int64_t batch, int64_t length, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t max_length, float scale, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* out[r, i] = silu(gate) * up in fp32, gate = gate_up[r, i], up = gate_up[r, I + i]
 * (bf16 inputs, the fused gate|up projection), silu(x) = x / (1 + exp(-x)).
 * Replaces: the SwiGLU product of QwenMLP.forward (src/qwen_int4/model.py:133-136). */
int qwen2_silu_mul(const void* gate_up, float* out, int64_t rows, int64_t intermediate, void* stream);

/* Bytes of workspace qwen2_lm_head needs for its argmax (one key per row
 * per workgroup; nothing in it survives a call); 0 for unsupported sizes.
 * Calls sharing a workspace must be ordered on one stream. */
int64_t qwen2_lm_head_workspace_bytes(int64_t rows, int64_t vocab, int64_t hidden);

/* Dense bf16 LM head of a decode step, with the greedy choice (a second,
 * one-workgroup-per-row launch on the same stream):
 *   logits[r, v] = bf16( sum_k x[r, k] * weight[v, k] )   (fp32 sums)
 *   argmax[r]    = the smallest v with the largest logits[r, v]
 *                  (NaN counts as the largest; -0 equals +0)
 * for x bf16 [rows, hidden], weight bf16 [vocab, hidden] (Qwen2's tied
 * embedding), logits bf16 [rows, vocab], argmax int64 [rows] or NULL (then
 * no workspace is needed).  rows <= 16, hidden a multiple of 128 and at most
 * 4096; x and weight 16-byte aligned, workspace 8-byte aligned.
 * Replaces: the tied lm_head projection of QwenInt4ForCausalLM
 *           (src/qwen_int4/model.py:217-218, :243-245) and the greedy choice
 *           logits[:, -1].argmax(dim=-1) (src/qwen_int4/generation.py:51). */
int qwen2_lm_head(const void* x, const void* weight, void* logits, int64_t* argmax, int64_t rows, int64_t vocab,
                  int64_t hidden, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_INT4_HIP_QWEN2_DECODE_H */
