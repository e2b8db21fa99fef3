/*
 * aether_ops.h — C ABI of the dense transformer ops on MI355X (gfx950).
 *
 * The reference's non-attention layers run these Metal kernels through its
 * Rust Ops engine:
 *   nexus-core/src/ops.metal:16-635   copy_buffer, embed_lookup, rms_norm, rope,
 *                                     matmul_f16, vecmat_f16, vecmat_scaled,
 *                                     silu_gate, add_residual, add_bias,
 *                                     matmul_scaled, causal_attention,
 *                                     multihead_attention, scale_f16
 *   nexus-core/src/ops.rs:166-462     the dispatch methods, called by
 *                                     InferenceEngine::forward_batch (inference.rs:456-634)
 * Each entry point below names the method it replaces and keeps its argument
 * order and meaning, with the engine first and a HIP stream last.  Pointers are
 * device pointers; f16 tensors are IEEE binary16 bit patterns (uint16_t).  The
 * calls are asynchronous on `hip_stream` (NULL is HIP's null stream): the
 * reference's batch mode (ops.rs:88-101, one command buffer per forward pass)
 * is a stream here, or a HIP graph captured from it.  A count of zero is a
 * no-op.  Every function returns AW_OK or a negative AW_E_* code of
 * aether_weaver.h, with the engine's last error describing the failure.
 *
 * Arithmetic is the reference's: f16 loads converted to fp32, fp32 sums and
 * products, one rounding to f16 (or fp32 for the scaled products) at the
 * store.  The products run on the matrix cores (v_mfma_f32_16x16x32_f16).
 */
#ifndef AETHER_OPS_H
#define AETHER_OPS_H

#include <stddef.h>
#include <stdint.h>

#include "aether_weaver.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Ops::copy_buffer (ops.rs:166-180, ops.metal:16-26): dst[dst_off + i] =
 * src[src_off + i] for i < count; offsets in f16 elements.  The two ranges
 * must not overlap. */
int aw_ops_copy_buffer(aw_engine* engine, const uint16_t* src, uint16_t* dst, uint32_t count, uint32_t src_off,
                       uint32_t dst_off, void* hip_stream);

/* Ops::embed_lookup (ops.rs:183-206, ops.metal:33-49): output[t][:] =
 * embed_table[token_ids[t]][:] for t < seq_len, rows of hidden_size.  Added:
 * vocab_size, the table's row count.  An id >= vocab_size writes a zero row
 * and sets the engine's device error (aw_engine_check_device_errors reports
 * "token id"); the reference reads past its table. */
int aw_ops_embed_lookup(aw_engine* engine, const uint32_t* token_ids, const uint16_t* embed_table, uint16_t* output,
                        uint32_t hidden_size, uint32_t seq_len, uint32_t vocab_size, void* hip_stream);

/* Ops::rms_norm (ops.rs:209-231, ops.metal:59-99): per token row of
 * hidden_size, output = f16(x * (1 / sqrt(mean(x^2) + eps)) * weight).
 * output may equal input. */
int aw_ops_rms_norm(aw_engine* engine, const uint16_t* input, const uint16_t* weight, uint16_t* output,
                    uint32_t hidden_size, uint32_t num_tokens, float eps, void* hip_stream);

/* Ops::rope (ops.rs:234-263, ops.metal:107-155), in place on
 * q [num_tokens][q_heads][head_dim] and k [num_tokens][kv_heads][head_dim]:
 * the pair (x[p], x[p + head_dim/2]) of every head of token t rotates by
 * angle = f32(start_position + t) * freq_p, freq_p = 1 / theta^(2p / head_dim)
 * (taken in double precision and rounded to fp32; cos and sin of the fp32
 * angle likewise).  head_dim must be even; k may be NULL when kv_heads is 0. */
int aw_ops_rope(aw_engine* engine, uint16_t* q, uint16_t* k, uint32_t num_tokens, uint32_t q_heads, uint32_t kv_heads,
                uint32_t head_dim, uint32_t start_position, float theta, void* hip_stream);

/* Ops::matmul (ops.rs:266-296; kernels vecmat_f16 ops.metal:232-271 for m = 1,
 * matmul_f16 :170-216 otherwise): output [m][n] = f16(a [m][k] . b [n][k]^T),
 * fp32 accumulation.  Every column is computed (the reference's m = 1 launch
 * covers half of them: 8 columns per 256-thread group against the kernel's 16). */
int aw_ops_matmul(aw_engine* engine, const uint16_t* a, const uint16_t* b, uint16_t* output, uint32_t m, uint32_t n,
                  uint32_t k, void* hip_stream);

/* Ops::matmul_scaled (ops.rs:366-406; vecmat_scaled ops.metal:279-318,
 * matmul_scaled :380-422): output [m][n] = (a . b^T) * scale in fp32 (the
 * logits of the lm_head). */
int aw_ops_matmul_scaled(aw_engine* engine, const uint16_t* a, const uint16_t* b, float* output, uint32_t m,
                         uint32_t n, uint32_t k, float scale, void* hip_stream);

/* Ops::silu_gate (ops.rs:299-312, ops.metal:325-338):
 * output[i] = f16(gate[i] / (1 + exp(-gate[i])) * up[i]). */
int aw_ops_silu_gate(aw_engine* engine, const uint16_t* gate, const uint16_t* up, uint16_t* output, uint32_t size,
                     void* hip_stream);

/* Ops::add_residual (ops.rs:315-327, ops.metal:345-353): x[i] = f16(x[i] + residual[i]). */
int aw_ops_add_residual(aw_engine* engine, uint16_t* x, const uint16_t* residual, uint32_t size, void* hip_stream);

/* Ops::add_bias (ops.rs:330-343, ops.metal:360-371): x[t][d] = f16(x[t][d] + bias[d]). */
int aw_ops_add_bias(aw_engine* engine, uint16_t* x, const uint16_t* bias, uint32_t hidden_size, uint32_t num_tokens,
                    void* hip_stream);

/* Ops::scale_f16 (ops.rs:350-363, ops.metal:627-635): x[i] = f16(x[i] * scale). */
int aw_ops_scale_f16(aw_engine* engine, uint16_t* x, uint32_t count, float scale, void* hip_stream);

/* Ops::causal_attention (ops.rs:409-430, ops.metal:435-518), the legacy
 * single-head attention: output [head_dim] = softmax(q . K^T / sqrt(head_dim)) V
 * over kv_len rows of k and v [rows][head_dim].  Runs as
 * aw_multihead_attention_device with one head and one query, so head_dim is 64
 * or 128 and k and v must hold cache_tokens >= kv_len rounded up to 16 rows
 * (the reference's kv_len <= 4096 limit does not apply). */
int aw_ops_causal_attention(aw_engine* engine, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            uint16_t* output, uint32_t kv_len, uint32_t head_dim, uint64_t cache_tokens,
                            void* hip_stream);

/* Ops::multihead_attention is aw_multihead_attention_device (aether_weaver.h). */

/* ---- fused forms (no reference counterpart) --------------------------------
 * Pairs and triples of the calls above that forward_batch makes back to back
 * (inference.rs:518-600), each in one launch, with the output bits of the
 * separate calls: a product's bits do not depend on how many products share a
 * launch (its K partial sums are added in a fixed order). */

/* aw_ops_matmul, aw_ops_scale_f16 of its output by residual_multiplier, then
 * aw_ops_add_residual of it into x (ops.rs:266-296, :350-363, :315-327; the
 * o_proj and down_proj steps, inference.rs:564-572,592-600):
 * p = f16(a . b^T), p = f16(p * residual_multiplier), x [m][n] = f16(x + p).
 * A multiplier of 1 (the reference skips the scale then) gives the same bits. */
int aw_ops_matmul_add_residual(aw_engine* engine, const uint16_t* a, const uint16_t* b, uint16_t* x, uint32_t m,
                               uint32_t n, uint32_t k, float residual_multiplier, void* hip_stream);

/* aw_ops_matmul with b_gate and with b_up, then aw_ops_silu_gate (ops.rs:266-312;
 * inference.rs:586-591): output [m][n] = f16(silu(f16(a . b_gate^T)) * f16(a . b_up^T)).
 * m <= 64 (decode and verify steps); larger m returns AW_E_UNSUPPORTED. */
int aw_ops_matmul_silu_gate(aw_engine* engine, const uint16_t* a, const uint16_t* b_gate, const uint16_t* b_up,
                            uint16_t* output, uint32_t m, uint32_t n, uint32_t k, void* hip_stream);

/* The three aw_ops_matmul calls of the q, k and v projections (inference.rs:518-523):
 * q [m][n_q] = a . b_q^T, k_out [m][n_kv] = a . b_k^T, v_out [m][n_kv] = a . b_v^T. */
int aw_ops_matmul_qkv(aw_engine* engine, const uint16_t* a, const uint16_t* b_q, const uint16_t* b_k,
                      const uint16_t* b_v, uint16_t* q, uint16_t* k_out, uint16_t* v_out, uint32_t m, uint32_t n_q,
                      uint32_t n_kv, uint32_t k, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* AETHER_OPS_H */
