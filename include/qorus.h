/*
 * qorus.h -- public C API of the Qorus-IA quantized matrix path, implemented
 * for AMD Instinct MI355X (gfx950) by libqorus_hip.so.
 *
 * Every entry point keeps the name, signature, argument meaning, validation
 * order and q_error_code returns of the reference declaration it replaces
 * (cited per function), so existing callers relink unchanged.  The op entry
 * points take HOST pointers and are synchronous, exactly like the reference:
 * inputs are copied to HBM, the gfx950 kernel runs, outputs are copied back.
 * Q4_0 views whose data lie inside a model mapped by q_init_memory[_ex] are
 * read from the HBM-resident copy made at load time, with no per-call copy.
 * The stream-ordered device entry points used by the on-device decode step
 * are declared in qorus_hip.h.
 *
 * The BPE tokenizer and q_generate are host code around the device path
 * (text in, token ids to the model, ids back to text).
 */
#ifndef QORUS_H
#define QORUS_H

#include "qorus_types.h"

#ifdef __cplusplus
#define Q_RESTRICT __restrict__
extern "C" {
#else
#define Q_RESTRICT restrict
#endif

/* ---- Memory tiers (reference include/qorus.h:16-39, src/core/memory.c) ---- */

/* Map a .qorus file (tier 1) and upload it once to HBM.
 * Replaces reference qorus.h:16 / memory.c:131-133. */
q_error_code q_init_memory(q_context* Q_RESTRICT ctx, const char* model_path);

/* As q_init_memory with an explicit host mapping strategy.
 * Replaces reference qorus.h:21 / memory.c:60-128. */
q_error_code q_init_memory_ex(q_context* Q_RESTRICT ctx, const char* model_path,
                              q_mmap_strategy strategy);

/* Allocate the tier-2 KV cache, zero-filled, in HBM (kv_buffer is a device
 * address).  Replaces reference qorus.h:25 / memory.c:136-164. */
q_error_code q_alloc_kv_cache(q_context* Q_RESTRICT ctx, size_t kv_size);

/* Allocate the tier-3 host arena (tensor views, model structs).
 * Replaces reference qorus.h:29 / memory.c:168-195. */
q_error_code q_alloc_arena(q_context* Q_RESTRICT ctx, size_t arena_size);

/* 64-byte aligned bump allocation; NULL on OOM.
 * Replaces reference qorus.h:33 / memory.c:199-259. */
void* q_arena_alloc(q_context* Q_RESTRICT ctx, size_t size);

/* Rewind the arena to the model watermark.
 * Replaces reference qorus.h:36 / memory.c:265-315. */
void q_arena_reset(q_context* Q_RESTRICT ctx);

/* Release arena, KV cache, HBM mirrors and mapping (LIFO).
 * Replaces reference qorus.h:39 / memory.c:317-355. */
void q_free_memory(q_context* Q_RESTRICT ctx);

/* Replaces reference qorus.h:47 / src/core/utils.c:11-31. */
const char* q_strerror(q_error_code err);

/* ---- Ops (host pointers, synchronous) ---- */

/* Dequantize one Q4_0 block into 32 floats; silent no-op on NULL.
 * Replaces reference qorus.h:58-61 / src/ops/avx2/dequantize.c:82-96. */
void q_dequantize_q4_0_block_avx2_public(const q_block_q4_0* Q_RESTRICT block,
                                         float* Q_RESTRICT output);

/* y[M] = W[M x N] . x[N] with Q4_0 W.
 * Replaces reference qorus.h:70-74 / src/ops/avx2/matmul.c:98-271. */
q_error_code q_gemv_q4_f32_avx2(const q_tensor* Q_RESTRICT weights,
                                const float* Q_RESTRICT input,
                                float* Q_RESTRICT output);

/* C[M x N] = A[M x K] . B[K x N], fp32; B may be a transposed view
 * (nb[0] == 4, ne[0] > 1, nb[1] > 4: element (k, j) at B->data[j*K + k]).
 * Same validation order and codes as the reference; a non-transposed B
 * takes N*K*4 bytes from ctx's arena (the reference's transpose buffer,
 * -> Q_ERR_ARENA_OOM when it does not fit).  Host pointers, synchronous;
 * every dot product follows the reference's accumulation order exactly.
 * Replaces reference qorus.h:84-89 / src/ops/avx2/matmul_fp32.c:57-474. */
q_error_code q_matmul_f32_avx2(const q_tensor* Q_RESTRICT A,
                               const q_tensor* Q_RESTRICT B, q_tensor* C,
                               q_context* Q_RESTRICT ctx);

/* Causal mask: every element above the diagonal of the square fp32 matrix
 * scores [n x n] (row stride nb[0]/4 >= n) := mask_value; the rest keeps
 * its bits.  Same validation order and codes as the reference.  Host
 * pointers, synchronous (the batched prefill of llama_forward needs no
 * mask: each query attends exactly the cached keys up to its position).
 * Replaces reference qorus.h:91-100 / src/ops/avx2/causal_mask_fp32.c:16-138. */
q_error_code q_causal_mask_f32_avx2(q_tensor* scores, float mask_value);

/* out = a + b (1-D, in-place allowed).
 * Replaces reference qorus.h:109-113 / src/ops/avx2/add_fp32.c:17-164. */
q_error_code q_add_f32_avx2(const q_tensor* a, const q_tensor* b, q_tensor* output);

/* out = a * b (1-D, in-place allowed).
 * Replaces reference qorus.h:122-126 / src/ops/avx2/mul_fp32.c:17-126. */
q_error_code q_mul_f32_avx2(const q_tensor* a, const q_tensor* b, q_tensor* output);

/* y = x * rsqrt(mean(x^2) + eps) * weight.
 * Replaces reference qorus.h:138-144 / src/ops/avx2/rmsnorm.c:15-92. */
q_error_code q_rmsnorm_f32_avx2(const float* Q_RESTRICT x, const float* Q_RESTRICT weight,
                                float* Q_RESTRICT output, uint32_t N, float eps);

/* Interleaved-pair rotation with duplicated cos/sin tables [c0,c0,c1,c1,...].
 * Replaces reference qorus.h:153-159 / src/ops/avx2/rope.c:23-110. */
q_error_code q_rope_f32_avx2(const float* Q_RESTRICT x, const float* Q_RESTRICT cos,
                             const float* Q_RESTRICT sin, float* Q_RESTRICT output,
                             uint32_t N);

/* y = x * sigmoid(x) with the reference's polynomial exp.
 * Replaces reference qorus.h:167-171 / src/ops/avx2/silu.c:18-94. */
q_error_code q_silu_f32_avx2(const float* Q_RESTRICT x, float* Q_RESTRICT output, uint32_t N);

/* Max-shifted softmax with the reference's polynomial exp.
 * Replaces reference qorus.h:179-183 / src/ops/avx2/softmax.c:17-132. */
q_error_code q_softmax_f32_avx2(const float* Q_RESTRICT x, float* Q_RESTRICT output, uint32_t N);

/* ---- Llama-3 model (reference include/qorus.h:193-219) ---- */

/* Build tensor views over the mapped model and the HBM decode plan.
 * Replaces reference qorus.h:193-196 / src/models/model.c:294-673. */
q_error_code llama_build_graph(q_context* Q_RESTRICT ctx, q_llama_model* Q_RESTRICT model);

/* Replaces reference qorus.h:200 / src/models/model.c:675-691. */
void llama_free_graph(q_llama_model* Q_RESTRICT model);

/* Run tokens[0..seq_len) at positions pos.. and write the logits of the
 * last token to the host buffer `logits` [vocab_size].
 * Replaces reference qorus.h:212-219 / src/models/model.c:1655-1850. */
q_error_code llama_forward(q_llama_model* Q_RESTRICT model, q_context* Q_RESTRICT ctx,
                           const uint32_t* Q_RESTRICT tokens, uint32_t seq_len,
                           uint32_t pos, float* Q_RESTRICT logits);

/* Next-token selection on the GPU, with the reference's validation order,
 * arena allocations and thread-local xorshift64* stream.  temperature <
 * 1e-6: greedy, the first index of the maximum.  Otherwise softmax of
 * logits / temperature in the reference's order, then top-k and/or top-p
 * filtering and one draw; equal probabilities at a top-k/top-p cut keep the
 * lower indices, and with neither filter every token is a candidate (two
 * cases the reference leaves to its sort internals or unwritten memory).
 * logits are host memory, as in the reference.
 * Replaces reference qorus.h:285-300 / src/main.c:852-992. */
q_error_code q_sample_token(const float* Q_RESTRICT logits, uint32_t vocab_size,
                            float temperature, uint32_t top_k, float top_p,
                            uint32_t* Q_RESTRICT token_id_out, q_context* Q_RESTRICT ctx);

/* Autoregressive generation: the prompt through llama_forward at position 0
 * (the batched prefill), then per step q_sample_token on the last logits
 * (with state->ctx's arena), the token stored, a stop at the tokenizer's EOS
 * or a full context, and the token through llama_forward at the next
 * position.  Same validation order and codes as the reference; the arena is
 * reset before each forward, as there.  (qh_llama_generate_sampled in
 * qorus_hip.h is the same loop with the sampling on device logits and no
 * EOS stop.)  Replaces reference qorus.h:302-320 / src/main.c:994-1131. */
q_error_code q_generate(q_generation_state* Q_RESTRICT state);

/* ---- BPE tokenizer (host; reference include/qorus.h:224-273,
 *      src/tokenizer/bpe.c) ---- */

/* Load a 'QTKR' v1 tokenizer file (32-byte header, length-prefixed vocab
 * strings, (id1, id2, merged) rules).  Same validation order and codes as
 * the reference.  Replaces reference qorus.h:226-230 / bpe.c:263-... */
q_error_code q_tokenizer_load(q_tokenizer* Q_RESTRICT tok, const char* tokenizer_path);

/* Text -> ids: one token per byte, the merge rules applied greedily in file
 * order until nothing changes, BOS/EOS on request; Q_ERR_ARENA_OOM when the
 * result exceeds max_tokens.  Replaces reference qorus.h:232-250 /
 * bpe.c:692-808. */
q_error_code q_tokenizer_encode(q_tokenizer* Q_RESTRICT tok, const char* Q_RESTRICT text,
                                uint32_t* Q_RESTRICT tokens_out, uint32_t* Q_RESTRICT num_tokens_out,
                                uint32_t max_tokens, bool add_bos, bool add_eos);

/* Ids -> text (special and out-of-vocabulary ids skipped; Q_ERR_ARENA_OOM
 * and a truncated text when the buffer is short).  Replaces reference
 * qorus.h:252-266 / bpe.c:811-866. */
q_error_code q_tokenizer_decode(q_tokenizer* Q_RESTRICT tok, const uint32_t* Q_RESTRICT tokens,
                                uint32_t num_tokens, char* Q_RESTRICT text_out, size_t text_buf_size);

/* Free what q_tokenizer_load allocated and zero the struct.
 * Replaces reference qorus.h:268-273 / bpe.c:869-887. */
void q_tokenizer_free(q_tokenizer* Q_RESTRICT tok);

#ifdef __cplusplus
}
#endif

#endif /* QORUS_H */
