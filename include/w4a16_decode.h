/*
 * W4A16 decode-step extensions for gfx950 (MI355X): the fused GEMV variants
 * and the small kernels that, together with the W4A16 linear layer, run one
 * greedy-decode step of a Llama-architecture model in 4 or 5 launches per
 * layer plus 2.
 *
 * Reference interfaces they replace (chris320211/Nibble): the reference runs
 * its end-to-end decode (scripts/generate.py:260-305, HF generate with a
 * static cache under CUDA graphs) through Hugging Face's Llama modules, whose
 * RMSNorm, rotary embedding, attention, SiLU-gated MLP, residual adds and
 * argmax are separate eager kernels around its w4a16::linear calls
 * (w4a16/linear.py:154-200). These entry points fuse those operations into
 * the GEMV's prologue / epilogue or into one kernel each; they have no
 * one-to-one counterpart in the reference's C++ (csrc/ holds only the
 * linear and dequantize ops).
 *
 * Conventions are those of w4a16_hip.h: device pointers, a hipStream_t
 * passed as void*, W4A16_OK or a W4A16_ERR_* code whose message
 * w4a16_last_error returns, nothing allocated or synchronised
 * (graph-capturable).
 */
#ifndef W4A16_DECODE_H
#define W4A16_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * One activation row (M = 1) through an INT4 linear layer with the decode
 * step's neighbouring element-wise work fused in:
 *   norm_weight != NULL: RMSNorm the row first (fp32 mean of squares,
 *     x * rsqrt(mean + eps) * norm_weight, rounded to fp16);
 *   paired == 0: output[n] = fp16(W[n] . x') (+ residual[n] in fp16 when
 *     residual != NULL; residual may alias output);
 *   paired != 0: W is [gate; up] with N rows (N even) and
 *     output[i] = fp16(silu(fp16(W[i] . x')) * fp16(W[i + N/2] . x')),
 *     i < N/2 (residual must be NULL).
 * Needs group_size 128, K a multiple of 128 up to 16384, and 16-byte aligned
 * activations, norm_weight and packed_weights.
 * Replaces (reference): Llama RMSNorm + q/k/v or gate/up QuantizedLinear
 * calls (w4a16/linear.py:154-200) + act_fn(gate) * up + residual add.
 */
int w4a16_gemv_fused_f16(const void* activations, const void* norm_weight, float eps,
                         const uint8_t* packed_weights, const void* scales,
                         const void* residual, void* output, int64_t N, int64_t K,
                         int64_t group_size, int paired, void* stream);

/*
 * The lm_head GEMV with the greedy argmax in its epilogue: logits[n] =
 * fp16(W[n] . x') as w4a16_gemv_fused_f16 (norm_weight optional; logits may
 * be NULL when the caller does not need them), then in the same launch
 * *token = first index of the maximum logit (a NaN counts as the maximum,
 * -0 as +0, as torch.argmax), *position += 1 when position != NULL, and
 * emb_out[0..hidden) = table[*token, :] when table / emb_out are given
 * (vocab >= N). Each workgroup publishes its best (logit, index) in the
 * workspace and the last one to arrive finishes the reduction.
 * workspace: device memory of at least w4a16_gemv_argmax_workspace_bytes(N)
 * bytes, 16-byte aligned, zero-filled once before its first use; every call
 * leaves its counters at zero again, so it is reused as is (also under graph
 * capture). Calls that share a workspace must not run concurrently.
 * Needs group_size 128, 0 < K <= 16384 (multiple of 128), 16-byte aligned
 * activations, norm_weight and packed_weights.
 * Cost on MI355X: each workgroup's device-scope release / acquire fences
 * write back and invalidate its XCD's L2 while the other workgroups stream
 * weights, ~30 ns per workgroup in series (61 us for a 32000 x 2048 lm_head
 * against 8.8 us + 6.8 us for w4a16_gemv_fused_f16 + w4a16_argmax_embed_f16),
 * so that pair stays the decode step's choice.
 * Replaces (reference): lm_head QuantizedLinear (w4a16/linear.py:154-200)
 * + the greedy pick of HF generate(do_sample=False) and the next step's
 * embedding lookup (scripts/generate.py:286-293).
 */
int64_t w4a16_gemv_argmax_workspace_bytes(int64_t N);
int w4a16_gemv_argmax_f16(const void* activations, const void* norm_weight, float eps,
                          const uint8_t* packed_weights, const void* scales, void* logits,
                          int64_t N, int64_t K, int64_t group_size, int64_t* token,
                          int64_t* position, const void* table, int64_t vocab, int64_t hidden,
                          void* emb_out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Attention of one new token at position *position (device int64):
 * qkv = [q (num_heads x 64) | k (num_kv_heads x 64) | v (num_kv_heads x 64)]
 * fp16; rotary embedding (half-split, cos / sin tables [max_seq_len, 32]
 * fp32) on q and k; k and v appended to the caches [num_kv_heads,
 * max_seq_len, 64] fp16 at the position; output [num_heads x 64] fp16 =
 * softmax(q k^T / 8) v over cache slots 0..position. head_dim must be 64.
 * A position outside [0, max_seq_len) writes NaN and leaves the caches alone.
 * Replaces (reference): HF LlamaAttention's rotary embedding, static-cache
 * update and sdpa call in the decode loop of scripts/generate.py:260-305.
 */
int w4a16_decode_attention_f16(const void* qkv, void* k_cache, void* v_cache,
                               const float* cos_table, const float* sin_table,
                               const int64_t* position, void* output,
                               int64_t num_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t max_seq_len, void* stream);

/*
 * w4a16_decode_attention_f16 with each head's slots 0 .. position split into
 * up to `splits` shares of whole 64-slot chunks (at least 192 slots each), one workgroup per head and share
 * (num_heads x splits workgroups, where the unsplit form has num_heads), then
 * a second launch that merges the shares' softmax states per head. workspace:
 * num_heads * splits * 66 fp32 (264 bytes per head and share, 4-byte
 * aligned), overwritten by every call; calls that share one must not run
 * concurrently. 1 <= splits <= 64; other arguments, output and NaN rows as
 * w4a16_decode_attention_f16 (the new k / v rows are appended once).
 * Replaces (reference): the same attention as w4a16_decode_attention_f16.
 */
int w4a16_decode_attention_split_f16(const void* qkv, void* k_cache, void* v_cache,
                                     const float* cos_table, const float* sin_table,
                                     const int64_t* position, void* output,
                                     int64_t num_heads, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t max_seq_len, int64_t splits,
                                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Attention of one new token fused with the o projection and the residual
 * add, for positions below 64 (one chunk of cache slots):
 *   attn = softmax(q k^T / 8) v as w4a16_decode_attention_f16 (same qkv
 *     layout, caches and append), except that cos / sin of
 *     position * inv_freq[i] (inv_freq: 32 fp32, i < 32) are computed in
 *     the kernel instead of read from tables;
 *   residual[n] = fp16(residual[n] + fp16(o_packed[n] . attn)), n < hidden,
 *     with the o projection [hidden, num_heads * 64] INT4 group 128.
 * Needs head_dim 64, num_kv_heads 1, 2, 4 or 8, num_heads / num_kv_heads <= 16,
 * num_heads * 64 <= 4096, group_size 128, 16-byte aligned qkv, caches and
 * o_packed. A position outside [0, min(max_seq_len, 64)) writes NaN to every
 * residual row and leaves the caches alone.
 * Replaces (reference): HF LlamaAttention (rotary, static-cache update,
 * sdpa) + o_proj QuantizedLinear + residual add of one decoder layer in the
 * decode loop of scripts/generate.py:260-305 (w4a16/linear.py:154-200 for
 * the o_proj call).
 */
int w4a16_attention_o_f16(const void* qkv, void* k_cache, void* v_cache, const float* inv_freq,
                          const int64_t* position, const uint8_t* o_packed, const void* o_scales,
                          void* residual, int64_t num_heads, int64_t num_kv_heads,
                          int64_t head_dim, int64_t max_seq_len, int64_t hidden,
                          int64_t group_size, void* stream);

/*
 * The q|k|v projection of a decode step with the rotary embedding and the
 * KV-cache append in its epilogue: qkv = W . x' as w4a16_gemv_fused_f16
 * (norm_weight optional), N = (num_heads + 2 num_kv_heads) * 64 rows in the
 * layout of w4a16_decode_attention_f16, each rounded to fp16; then every q
 * and k head's dims (d, d + 32), d < 32, are rotated by the fp32 angle
 * position * inv_freq[d] (fp32 products of the fp16 values, rounded to
 * fp16), the rotated q and k and the v rows are stored in qkv, and when
 * 0 <= position < max_seq_len the k and v rows go to cache slot `position`
 * of k_cache / v_cache [num_kv_heads, max_seq_len, 64] (other slots are not
 * touched). Needs head_dim 64, group_size 128, K a multiple of 128 up to
 * 16384, 16-byte aligned activations, norm_weight and packed_weights.
 * Replaces (reference): Llama input RMSNorm + q_proj / k_proj / v_proj
 * QuantizedLinear calls (w4a16/linear.py:154-200) + rotary embedding +
 * static-cache update of HF LlamaAttention in scripts/generate.py:260-305.
 */
int w4a16_gemv_qkv_rope_f16(const void* activations, const void* norm_weight, float eps,
                            const uint8_t* packed_weights, const void* scales, void* qkv,
                            void* k_cache, void* v_cache, const float* inv_freq,
                            const int64_t* position, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t max_seq_len, int64_t K,
                            int64_t group_size, void* stream);

/*
 * w4a16_attention_o_f16 after w4a16_gemv_qkv_rope_f16: q in qkv is already
 * rotated and slot `position` of the caches already holds the new k and v,
 * so the kernel only reads them (k and v in qkv are not used): residual[n] =
 * fp16(residual[n] + fp16(o_packed[n] . attn)), attn = softmax(q k^T / 8) v
 * over cache slots 0..position. Same requirements and out-of-range
 * behaviour as w4a16_attention_o_f16 (NaN rows, caches untouched).
 * Replaces (reference): as w4a16_attention_o_f16, without the rotary
 * embedding and cache update.
 */
int w4a16_attention_o_cached_f16(const void* qkv, const void* k_cache, const void* v_cache,
                                 const int64_t* position, const uint8_t* o_packed,
                                 const void* o_scales, void* residual, int64_t num_heads,
                                 int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len,
                                 int64_t hidden, int64_t group_size, void* stream);

/*
 * Greedy token: *token = first index of the maximum of logits[0..n) (fp16),
 * with torch.argmax's special values: any NaN counts as the largest value
 * (the first NaN wins), -0 equals +0, all -inf gives 0; if position != NULL,
 * *position += 1.
 * Replaces (reference): the greedy pick of HF generate(do_sample=False),
 * scripts/generate.py:286-293.
 */
int w4a16_argmax_f16(const void* logits, int64_t n, int64_t* token, int64_t* position,
                     void* stream);

/*
 * w4a16_argmax_f16, then output[0..hidden) = table[*token, :] (fp16 [vocab,
 * hidden], vocab >= n): the next step's embedding gathered by the same
 * launch, so a decode step needs no separate gather. token_copy (may be
 * NULL) receives the token too: a slot of a caller's token history (a graph
 * of several decode steps gives each step's launch its own slot, so no copy
 * launch follows the step).
 * Replaces (reference): the greedy pick plus the next step's embedding
 * lookup (scripts/generate.py:286-293).
 */
int w4a16_argmax_embed_f16(const void* logits, int64_t n, int64_t* token, int64_t* position,
                           const void* table, int64_t vocab, int64_t hidden, void* output,
                           int64_t* token_copy, void* stream);

/*
 * x_out[r, :] = table[tokens[r], :] (fp16 [vocab, hidden]; zeros for a token
 * outside [0, vocab)) and output[r, :] = RMSNorm(x_out[r, :]) * weight for
 * r < rows, one launch: the prompt's embedding rows and the first layer's
 * input RMSNorm (the arithmetic of w4a16_rmsnorm_f16, bit for bit); position
 * (int64[1], may be NULL) <- rows, the decode position after the prompt.
 * hidden a multiple of 8 up to 8192; table, weight, x_out and output 16-byte
 * aligned; tokens int64 [rows]. rows = 0 launches nothing (the position is
 * left as it was).
 * Replaces (reference): the prompt's embedding lookup and the first input
 * RMSNorm of HF's Llama forward (scripts/generate.py:260-305).
 */
int w4a16_embed_rmsnorm_f16(const void* table, int64_t vocab, int64_t hidden, const int64_t* tokens,
                            int64_t rows, const void* weight, float eps, void* x_out, void* output,
                            int64_t* position, void* stream);

/*
 * output[0..hidden) = table[*token, :] (fp16 [vocab, hidden]); a token
 * outside [0, vocab) gives zeros.
 * Replaces (reference): the embedding lookup of the decode step.
 */
int w4a16_embedding_f16(const void* table, int64_t vocab, int64_t hidden,
                        const int64_t* token, void* output, void* stream);

/*
 * Prefill of a T-token prompt: the element-wise work between its W4A16
 * projections, one launch each (replaces the torch ops of HF LlamaModel's
 * prefill forward around the reference's w4a16::linear / dequantize calls,
 * scripts/generate.py:260-305 with w4a16/linear.py:154-200).
 *
 * RMSNorm of `rows` rows of `hidden` fp16: output[r] = fp16((fp32(x[r]) *
 * inv) * fp32(weight)), inv = 1 / sqrt(mean(x[r]^2) + eps) in fp32 (the
 * arithmetic of w4a16_gemv_fused_f16's prologue).
 */
int w4a16_rmsnorm_f16(const void* x, const void* weight, float eps, void* output, int64_t rows, int64_t hidden,
                      void* stream);

/*
 * output[r, i] = fp16(fp16(silu(g)) * u) for g = gate_up[r, i] and u =
 * gate_up[r, inter + i] (rows of [gate | up], 2 * inter wide; the roundings
 * of silu(g) * u on fp16 tensors).
 */
int w4a16_silu_mul_f16(const void* gate_up, void* output, int64_t rows, int64_t inter, void* stream);

/*
 * SiLU-gated projection: output[m, i] = fp16(fp16(silu(g)) * u) with g =
 * (activations @ W[i]^T) and u = (activations @ W[inter + i]^T) each rounded
 * to fp16, for packed_weights [2 inter, K / 2] and scales [2 inter, K / 128]
 * holding the gate rows then the up rows. The same values as
 * w4a16_linear_f16 over the 2 inter rows followed by w4a16_silu_mul_f16, in
 * one launch: the W4A16 GEMM with the multiply in its epilogue (M >= 2, or
 * K > 16384; M = 9..16 on rows longer than 4096 weights, or on 2 inter >=
 * 8192 rows of up to 2048, where the 16-row-slot paired plan stages whole
 * rows: that kernel's SiLU form), or the decode step's
 * paired fused GEMV (M = 1). Replaces the
 * gate_proj / up_proj QuantizedLinear calls and act_fn(gate) * up of HF's
 * LlamaMLP (w4a16/linear.py:154-200 for each projection). Needs group_size
 * 128, 16-byte aligned activations and weights, operands below 4 GiB.
 */
int w4a16_linear_silu_f16(const void* activations, const uint8_t* packed_weights, const void* scales, void* output,
                          int64_t M, int64_t inter, int64_t K, int64_t group_size, void* stream);

/*
 * Residual add + RMSNorm over `rows` rows of `hidden` fp16 values (hidden <=
 * 8192): x_out = fp16(x + delta) (an fp16 tensor add's rounding), output =
 * RMSNorm(x_out) * weight as w4a16_rmsnorm_f16 computes it. x_out may be x.
 * Replaces the prefill's "x + linear(a)" followed by the next RMSNorm
 * (HF LlamaDecoderLayer's residual adds and post_attention_layernorm /
 * the next layer's input_layernorm, scripts/generate.py:260-305).
 */
int w4a16_add_rmsnorm_f16(const void* x, const void* delta, const void* weight, float eps, void* x_out,
                          void* output, int64_t rows, int64_t hidden, void* stream);

/*
 * A linear layer followed by the residual add + RMSNorm of its output rows
 * (the down projection of a prompt and the next layer's input norm):
 * x_out = fp16(x + linear(activations)) and output = RMSNorm(x_out) *
 * norm_weight, bit-identical to w4a16_linear_ws_f16 followed by
 * w4a16_add_rmsnorm_f16. Where the op takes the ring kernel's K slices on
 * rows of at most 2048 outputs, the slices' sum runs in the norm's launch
 * (two launches instead of three). workspace (16-byte aligned) holds
 * w4a16_linear_add_rmsnorm_workspace_bytes(M, N, K, group_size) bytes:
 * split-K partial sums, then an fp16 copy of the linear's output. x_out may
 * be x. The decoder's fused prefill (reference w4a16/linear.py:154-200 for
 * the projection, the norms of its Llama blocks) calls it; no other
 * reference counterpart.
 */
int w4a16_linear_add_rmsnorm_f16(const void* activations, const uint8_t* packed_weights, const void* scales,
                                 const void* x, const void* norm_weight, float eps, void* x_out, void* output,
                                 int64_t M, int64_t N, int64_t K, int64_t group_size, void* workspace,
                                 int64_t workspace_bytes, void* stream);
int64_t w4a16_linear_add_rmsnorm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size);

/*
 * One layer's attention half of a prompt after its q|k|v projection: attn =
 * w4a16_prefill_attention_f16(qkv, caches, start, tokens) (which appends the
 * tokens' rotary k and v rows to the caches), then x_out = fp16(x +
 * linear(attn, o_packed, o_scales)) and output = RMSNorm(x_out) *
 * norm_weight as w4a16_linear_add_rmsnorm_f16 (K = num_heads * head_dim, N =
 * hidden). Where the o op runs one group
 * pair per wavefront on 16 row slots (9..16 tokens, K = 2048; start +
 * tokens <= 32, query heads per KV head a power of two, hidden <= 2048,
 * 16-byte aligned buffers, 4-byte aligned o_scales) the attention runs
 * inside the o projection's launch: each
 * workgroup attends the four query heads of its K slice and the norm's
 * launch sums the slices (two launches instead of three), with the
 * separate launches' arithmetic (the same MFMA chains per group pair, added
 * in the same order) up to the fp16 rounding of the fp32 rotary k and q,
 * which may differ by one unit; otherwise the separate launches. workspace
 * (16-byte aligned) holds
 * w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes(tokens, num_heads,
 * hidden, group_size) bytes. x_out may be x. The decoder's fused prefill
 * calls it (reference w4a16/linear.py:154-200 for the o projection, HF
 * LlamaAttention and the post-attention norm around it,
 * scripts/generate.py:260-305); no other reference counterpart.
 */
int w4a16_prefill_attention_o_add_rmsnorm_f16(const void* qkv, void* k_cache, void* v_cache, const float* cos_table,
                                              const float* sin_table, int64_t start, int64_t tokens,
                                              int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                              int64_t max_seq_len, const uint8_t* o_packed, const void* o_scales,
                                              int64_t hidden, int64_t group_size, const void* x,
                                              const void* norm_weight, float eps, void* x_out, void* output,
                                              void* workspace, int64_t workspace_bytes, void* stream);
int64_t w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes(int64_t tokens, int64_t num_heads, int64_t hidden,
                                                              int64_t group_size);

/*
 * Attention of `tokens` new tokens at cache slots start .. start + tokens - 1:
 * qkv rows [q (num_heads x 64) | k (num_kv_heads x 64) | v] fp16 as for
 * w4a16_decode_attention_f16; rotary embedding (cos / sin tables [max_seq_len,
 * 32] fp32) on q and k rounded to fp16; k and v appended to the caches; query t
 * attends to slots 0 .. start + t (slots below start read from the caches):
 * output[t] = softmax(q k^T / 8) v, [tokens, num_heads * 64] fp16.
 * Needs head_dim 64, start + tokens <= max_seq_len, 16-byte aligned caches.
 * When num_heads / num_kv_heads is a power of two up to 64 and qkv and the
 * tables are 16-byte aligned: the matrix cores, a workgroup per KV head and
 * 64 / group tokens (fp32 scores and an online softmax, the probabilities
 * rounded to fp16 for the value product). Up to 256 slots one launch, which
 * also appends its own tokens' rows to the caches; past 256 slots a launch
 * before it writes the new rotary k and v rows to the caches and the
 * attention streams the slots through LDS in blocks of 256. Otherwise (only
 * up to 256 slots; more return W4A16_ERR_SHAPE) one workgroup per query head
 * and block of 4 tokens (fp32 throughout); above 16 tokens a launch before
 * it writes the new rotary k and v rows to the caches.
 */
int w4a16_prefill_attention_f16(const void* qkv, void* k_cache, void* v_cache, const float* cos_table,
                                const float* sin_table, int64_t start, int64_t tokens, void* output,
                                int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_DECODE_H */
