/*
 * qorus_hip.h -- stream-ordered DEVICE entry points of libqorus_hip.so.
 *
 * These are the MI355X-native counterparts of the qorus.h ops: every pointer
 * argument is a device (HBM) address, every call is asynchronous on the given
 * stream (NULL = the null stream) and returns after validating its arguments
 * and enqueuing its kernels.  Validation order and q_error_code values follow
 * the reference op each entry point mirrors (cited per function); a kernel
 * launch failure is reported as Q_ERR_INVALID_ARG with the HIP message
 * available from qh_last_error().
 *
 * No CPU fallback exists: with no usable gfx950 device every entry point
 * returns Q_ERR_ALLOC_FAILED.
 */
#ifndef QORUS_HIP_H
#define QORUS_HIP_H

#include "qorus_types.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef void* qh_stream; /* a hipStream_t */
typedef void* qh_event;  /* a hipEvent_t */

/* ---- Runtime plumbing (no reference counterpart: the reference is CPU-only) ---- */

/* 1 if a GPU is visible and the library's device state initialised. */
int qh_available(void);
/* Text of the last HIP failure seen by the library ("" if none). */
const char* qh_last_error(void);
/* gfx architecture name of the current device, e.g. "gfx950". */
const char* qh_arch_name(void);

q_error_code qh_malloc(void** ptr, size_t bytes);
q_error_code qh_free(void* ptr);
/* Synchronous copies (host memory may be pageable). */
q_error_code qh_memcpy_htod(void* dst, const void* src, size_t bytes);
q_error_code qh_memcpy_dtoh(void* dst, const void* src, size_t bytes);
q_error_code qh_memcpy_dtod(void* dst, const void* src, size_t bytes, qh_stream s);
q_error_code qh_memset(void* dst, int value, size_t bytes, qh_stream s);
q_error_code qh_stream_create(qh_stream* s);
q_error_code qh_stream_destroy(qh_stream s);
q_error_code qh_stream_synchronize(qh_stream s);
q_error_code qh_device_synchronize(void);
q_error_code qh_event_create(qh_event* e);
q_error_code qh_event_destroy(qh_event e);
q_error_code qh_event_record(qh_event e, qh_stream s);
q_error_code qh_event_synchronize(qh_event e);
q_error_code qh_event_elapsed_ms(qh_event start, qh_event stop, float* ms);

/* HIP graphs: capture the work enqueued on stream s between begin and end
 * (by this thread) into an executable graph, then replay it. */
typedef void* qh_graph; /* a hipGraphExec_t */
q_error_code qh_stream_begin_capture(qh_stream s);
q_error_code qh_stream_end_capture(qh_stream s, qh_graph* out);
q_error_code qh_graph_launch(qh_graph g, qh_stream s);
q_error_code qh_graph_destroy(qh_graph g);

/* ---- Q4_0 dequantization and GEMV ---- */

/* out[32*b + e] = fmaf(q_e, s_b, -8*s_b) for b < n_blocks (bit-exact with
 * reference src/ops/avx2/dequantize.c:18-73).  out must be 16-byte aligned. */
q_error_code qh_dequantize_q4_0(const void* blocks, float* out, uint64_t n_blocks, qh_stream s);

/* Bytes of workspace qh_gemv_q4_f32 may use for an input of length N (it
 * only touches it when N > 16384; narrower inputs are converted inside the
 * GEMV launch). */
size_t qh_gemv_workspace_bytes(uint32_t N);

/* y[M] = W[M x N] . x[N], W->data in HBM (AoS 20-byte Q4_0 blocks, 4-byte
 * aligned), x/y 32-byte aligned.  Validation order and codes of reference
 * src/ops/avx2/matmul.c:104-197, plus Q_ERR_MISALIGNED for a W->data that
 * is not 4-byte aligned.  `workspace` holds >= qh_gemv_workspace_bytes(N)
 * device bytes; NULL selects a library-owned per-device buffer (calls that
 * overlap on one device then race on it).  Result: within 1e-5 of the fp64
 * dot product relative to sum_j |W_ij x_j| (an input that puts 7 or more
 * outliers of similar size in a block, each meeting a zero weight, is
 * outside this bound; see below).  x enters as integers with one
 * power-of-two scale per 32-element block (23-24 significant bits for the
 * block maximum); a block where a few outliers set that scale (removing
 * some 6 of its elements would leave less than 3/64 of its maximum) gets a
 * second 23-bit level, so every element within 2^21 of its block maximum
 * is exact.  Measured at the Llama-3 shapes: 0.4-2e-8 with N(0,1) x, and
 * the same with 1..6 equal outliers of 1e3..1e5 per block, or mixed sizes,
 * on zero weights, at or below the reference AVX2 order's error.  A block
 * left on level 1 keeps at least 3/64 of its maximum outside any 6 of its
 * elements; 8 equal outliers of 1e4 in every block on zero weights reach
 * about 2e-5 (CPU emulation of the digits). */
q_error_code qh_gemv_q4_f32(const q_tensor* W, const float* x, float* y, void* workspace,
                            qh_stream s);

/* y = W . x + residual (residual added last, as reference model.c:1620). */
q_error_code qh_gemv_q4_f32_add(const q_tensor* W, const float* x, const float* residual,
                                float* y, void* workspace, qh_stream s);

/* Split form of the GEMV for inputs shared by several matrices (fused Q|K|V
 * or gate|up in the decode step; no reference counterpart, the reference
 * calls q_gemv_q4_f32_avx2 once per matrix, model.c:1120-1165).
 * qh_gemv_prepare converts x (N floats, 32-byte aligned) into the integer
 * digit planes the kernel consumes, in `workspace`; qh_gemv_q4_f32_prepared
 * then computes ys[i] = Ws[i] . x (+ residuals[i] when residuals and
 * residuals[i] are non-NULL) for 1 <= n <= 4 matrices with the same N, in
 * one launch.  Each Ws[i] is validated as in qh_gemv_q4_f32. */
q_error_code qh_gemv_prepare(const float* x, uint32_t N, void* workspace, qh_stream s);
q_error_code qh_gemv_q4_f32_prepared(const q_tensor* const* Ws, const float* const* residuals,
                                     float* const* ys, uint32_t n, const void* workspace,
                                     qh_stream s);

/* ys[i] = Ws[i] . x (+ residuals[i]) for 1 <= n <= 4 matrices with the same
 * N, straight from the fp32 x: one launch for N <= 16384 (the digit planes
 * are made inside the GEMV), prepare + GEMV above that (`workspace` as in
 * qh_gemv_q4_f32, NULL for the library-owned buffer).  Each Ws[i], x and
 * ys[i] are validated as in qh_gemv_q4_f32; ys[i] must not overlap x.
 * Results are bit-identical to qh_gemv_prepare + qh_gemv_q4_f32_prepared.
 * No reference counterpart (the reference calls q_gemv_q4_f32_avx2 once per
 * matrix, src/models/model.c:1120-1165). */
q_error_code qh_gemv_q4_f32_multi(const q_tensor* const* Ws, const float* const* residuals,
                                  float* const* ys, uint32_t n, const float* x, void* workspace,
                                  qh_stream s);

/* ---- Batched prefill GEMM (MFMA) ----
 * Y[t][m] = sum_k W[m][k] * X[t][k] for t < T: the prefill projections of
 * reference src/models/model.c:1120-1165, 1446-1458, 1485-1512, 1555-1561,
 * which run q_gemv_q4_f32_avx2 (src/ops/avx2/matmul.c:98-271) once per
 * token row; here one MFMA contraction over all T rows.  X is [T][N]
 * row-major fp32 (16-byte aligned), Y is [T][M] fp32 (4-byte aligned, not
 * overlapping X).  Accuracy: max |Y - Y64| / sum_k |W x| at or below the
 * reference AVX2 order's (fp16 matrix cores with exact Q4 operands, a
 * two-part split of X and fp32 per-block scaling).  A token row holding a
 * non-finite value yields NaN outputs.
 * Validation, per matrix and in this order: W, X or Y NULL -> INVALID_ARG;
 * X not 16-byte or Y not 4-byte aligned -> MISALIGNED; M == 0, N == 0,
 * N % 32, N > 32768, N differing between the matrices or T == 0 ->
 * INVALID_SIZE;
 * type != Q4_0 -> INVALID_DTYPE; N/32 > UINT32_MAX/M or M*N/32*20 >= 2^31
 * -> OVERFLOW; nb[0] != N/32*20 or W->data NULL -> INVALID_ARG; W->data
 * not 4-byte aligned -> MISALIGNED; Y overlapping X -> ALIASING; then
 * workspace NULL -> INVALID_ARG.
 * `workspace` holds qh_gemm_workspace_bytes(N, T, M) bytes (for _multi:
 * M = sum of the matrices' rows). */
size_t qh_gemm_workspace_bytes(uint32_t N, uint32_t T, uint32_t M_total);
q_error_code qh_gemm_q4_f32(const q_tensor* W, const float* X, uint32_t T, float* Y, void* workspace,
                            qh_stream s);
/* Up to three matrices with the same N sharing X (Wq|Wk|Wv of attention,
 * W_gate|W_up of the MLP) in one launch: Ys[i] = X . Ws[i]^T, n in {1, 2, 3}. */
q_error_code qh_gemm_q4_f32_multi(const q_tensor* const* Ws, float* const* Ys, uint32_t n, const float* X,
                                  uint32_t T, void* workspace, qh_stream s);

/* ---- Vector ops (device pointers, same validation as the qorus.h op) ---- */

/* Device form of q_causal_mask_f32_avx2 (reference
 * src/ops/avx2/causal_mask_fp32.c:16-138): elements above the diagonal of
 * the n x n matrix at scores (row stride ld >= n floats) := mask_value.
 * scores NULL -> INVALID_ARG; n == 0 or ld < n -> INVALID_SIZE; not device
 * memory covering the n rows -> INVALID_ARG. */
q_error_code qh_causal_mask_f32(float* scores, uint32_t n, uint32_t ld, float mask_value, qh_stream s);

/* Reference src/ops/avx2/rmsnorm.c:15-92 (sum of squares reduced as a fixed
 * tree; the reference's 8-lane sequential order and rsqrtps seed are not
 * reproduced bit-for-bit). */
q_error_code qh_rmsnorm_f32(const float* x, const float* weight, float* output, uint32_t N,
                            float eps, qh_stream s);
/* Reference src/ops/avx2/rope.c:23-110 applied to n_vec consecutive vectors
 * of length N (e.g. all heads of a token) with one table pair; bit-exact. */
q_error_code qh_rope_f32(const float* x, const float* cos, const float* sin, float* output,
                         uint32_t N, uint32_t n_vec, qh_stream s);
/* Reference src/ops/avx2/silu.c:18-94; bit-exact on the first N&~7 elements. */
q_error_code qh_silu_f32(const float* x, float* output, uint32_t N, qh_stream s);
/* silu(gate) * up, the SwiGLU product of reference model.c:1516-1549. */
q_error_code qh_silu_mul_f32(const float* gate, const float* up, float* output, uint32_t N,
                             qh_stream s);
/* Reference src/ops/avx2/softmax.c:17-132 in its summation order (eight
 * lane sums over the first N&~7 elements, their fixed tree, then the tail
 * in index order, times 1/sum): bit-exact with q_softmax_f32_avx2 where the
 * tail's libm expf agrees with the device's (always when N % 8 == 0).
 * x may alias output.  The partial results live in a workspace:
 * qh_softmax_f32 uses one library workspace per process (calls that may
 * overlap on different streams must use qh_softmax_f32_ws with a workspace
 * of qh_softmax_workspace_bytes(N) device bytes each). */
q_error_code qh_softmax_f32(const float* x, float* output, uint32_t N, qh_stream s);
size_t qh_softmax_workspace_bytes(uint32_t N);
q_error_code qh_softmax_f32_ws(const float* x, float* output, uint32_t N, void* workspace, qh_stream s);
q_error_code qh_add_f32(const float* a, const float* b, float* output, uint32_t N, qh_stream s);
q_error_code qh_mul_f32(const float* a, const float* b, float* output, uint32_t N, qh_stream s);
/* Greedy argmax of reference src/main.c:870-881 (first index of the
 * maximum); writes the index to device memory *index_out.  Workspace rules
 * as for softmax (qh_argmax_f32_ws / qh_argmax_workspace_bytes). */
q_error_code qh_argmax_f32(const float* x, uint32_t N, uint32_t* index_out, qh_stream s);
size_t qh_argmax_workspace_bytes(uint32_t N);
q_error_code qh_argmax_f32_ws(const float* x, uint32_t N, uint32_t* index_out, void* workspace, qh_stream s);
/* Softmax of x into output and the greedy argmax of x into *index_out in
 * one pass structure (no reference counterpart: the reference's LM-head
 * step runs q_softmax_f32_avx2 and the argmax of src/main.c:870-881 one
 * after the other).  The index is the reference's; the softmax sums as a
 * tree over many workgroups, so the probabilities match the reference's
 * within 2e-6 relative (same zero pattern), not to the bit: the
 * exact-order qh_softmax_f32 runs its lane sums in one wave.  workspace holds
 * qh_softmax_workspace_bytes(N) device bytes; x must not alias output
 * (Q_ERR_ALIASING). */
q_error_code qh_softmax_argmax_f32_ws(const float* x, float* output, uint32_t N, uint32_t* index_out,
                                      void* workspace, qh_stream s);

/* LM head + softmax + greedy argmax: logits = W . x (as qh_gemv_q4_f32),
 * probs = softmax(logits) and *index_out = argmax(logits) (as
 * qh_softmax_argmax_f32_ws: the same bits and index; the probabilities are
 * its tree-sum form).  For 2048 < N <= 4096
 * and M >= 16384 the GEMV also leaves the argmax's per-workgroup partials,
 * so no separate pass re-reads the logits (3 launches).  workspace holds
 * qh_gemv_softmax_workspace_bytes(M) device bytes; probs must not alias
 * logits or x (Q_ERR_ALIASING).  No reference counterpart (the reference's
 * generation loop runs the LM head inside llama_forward, then
 * q_softmax_f32_avx2 and the argmax of src/main.c:870-881). */
size_t qh_gemv_softmax_workspace_bytes(uint32_t M);
q_error_code qh_gemv_q4_f32_softmax_argmax(const q_tensor* W, const float* x, float* logits, float* probs,
                                           uint32_t* index_out, void* workspace, qh_stream s);

/* qh_gemv_q4_f32_softmax_argmax without a workspace argument and without
 * any device allocation: its partials live in a 32 KB array in the
 * library's device memory, one per GPU, held until the process ends.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same results, bits and validation as the workspace form,
 * plus: N > 16384 (an input wider than the in-kernel digit conversion,
 * which would need a digit workspace) -> Q_ERR_INVALID_SIZE.  Every M fits
 * (the partials of at most 1024 slices, about 25 KB).  Nothing in the array
 * needs to start at zero (every partial is written before it is read within
 * a call), but calls that overlap on one GPU share the array and race:
 * serialize them (one stream, or events between streams). */
q_error_code qh_gemv_q4_f32_softmax_argmax_noalloc(const q_tensor* W, const float* x, float* logits,
                                                   float* probs, uint32_t* index_out, qh_stream s);

/* ---- Decode on the device ---- */

/* Greedy generation with no host round trip between steps (no reference
 * counterpart; it is the device form of the q_generate loop, reference
 * src/main.c:994-1131, with temperature 0): n_steps decode steps of a model
 * built by llama_build_graph, starting from `token` at position `pos`; each
 * step's argmax becomes the next token and the position advances on the
 * device.  tokens_out (host) receives the n_steps generated tokens and
 * *ms_per_step (if non-NULL) the mean step time from HIP events around the
 * replays of the captured step graph.  Requires pos + n_steps <= max_seq_len.
 * The KV cache rows pos..pos+n_steps-1 are overwritten. */
q_error_code qh_llama_generate(q_llama_model* model, q_context* ctx, uint32_t token, uint32_t pos,
                               uint32_t n_steps, uint32_t* tokens_out, float* ms_per_step);

/* Sampled generation on the device (no reference counterpart; the device
 * form of the q_generate loop, reference src/main.c:994-1131): as
 * qh_llama_generate, but each step's token is drawn by q_sample_token's
 * device pipeline (temperature, top_k, top_p with its semantics and
 * validation) from the logits in HBM, one draw of the calling thread's
 * sampling RNG per step.  The tokens equal a host loop of llama_forward and
 * q_sample_token on the same thread with 32-byte-aligned logits.
 * temperature < 1e-6 is qh_llama_generate. */
q_error_code qh_llama_generate_sampled(q_llama_model* model, q_context* ctx, uint32_t token, uint32_t pos,
                                       uint32_t n_steps, float temperature, uint32_t top_k, float top_p,
                                       uint32_t* tokens_out, float* ms_per_step);

/* ---- Sampling ---- */

/* q_sample_token (qorus.h; reference src/main.c:852-992) runs on the GPU:
 * temperature softmax, top-k, top-p and the CDF draw with the reference's
 * arithmetic, validation and arena use.  Its uniform draws come from a
 * per-thread xorshift64* state that starts at 123456789, as the
 * reference's.  These two calls set and read the calling thread's state
 * (no reference counterpart: the reference's state is private; they make a
 * sampled run reproducible). */
void qh_sample_set_state(uint64_t state);
uint64_t qh_sample_get_state(void);

#ifdef __cplusplus
}
#endif

#endif /* QORUS_HIP_H */
