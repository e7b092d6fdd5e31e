/*
 * qorus_oracle.h -- CPU ORACLE for the Qorus-IA quantized matrix path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library (project-ia_amd/)
 * links, loads or calls this code; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, always as the checker.
 *
 * Each function restates one reference routine in plain scalar C with the
 * reference's exact arithmetic order (FMA where the reference uses FMA,
 * separate rounding everywhere else; the file is built with
 * -ffp-contract=off, matching the reference's ISO -std=c11 build).  The
 * reference file:line each function follows is given at its definition.
 *
 * Parity status of each function (how it is pinned) is listed in
 * qorus_oracle.c's header.
 */
#ifndef QORUS_ORACLE_H
#define QORUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Q4_0: 20-byte blocks {qs[16], f32 scale}. */
void or_dequant_block(const uint8_t* blk, float out[32]);
void or_dequant_blocks(const uint8_t* blks, uint64_t n_blocks, float* out);

/* Threads used by the GEMV row loops and the attention heads (default 1;
 * results are the same bits for any count). */
void or_set_threads(int n);

/* GEMV in the reference AVX2 accumulation order; W is M x N, N % 32 == 0. */
void or_gemv_q4(const uint8_t* W, uint32_t M, uint32_t N, const float* x, float* y);
/* Same, rows [r0, r1) only (y indexed by absolute row). */
void or_gemv_q4_rows(const uint8_t* W, uint32_t r0, uint32_t r1, uint32_t N,
                     const float* x, float* y);
/* fp64 reference: y64 = sum_j ((q-8)*s) * x (exact dequant in double), and
 * cond = sum_j |((q-8)*s) * x|, the condition denominator. */
void or_gemv_q4_f64(const uint8_t* W, uint32_t M, uint32_t N, const float* x,
                    double* y64, double* cond);

/* RMSNorm with the reference's lane order; the reciprocal square root seed
 * is 1/sqrtf (the reference's rsqrtps seed is CPU-specific). */
void or_rmsnorm(const float* x, const float* w, float* y, uint32_t N, float eps);
void or_rope(const float* x, const float* cos_t, const float* sin_t, float* y, uint32_t N);
void or_rope_tables(float base, uint32_t head_dim, uint32_t pos, float* cos_t, float* sin_t);
float or_exp_approx(float x);
void or_silu(const float* x, float* y, uint32_t N);
void or_softmax(const float* x, float* y, uint32_t N);
uint32_t or_argmax(const float* x, uint32_t N);
/* q_sample_token, temperature > 0 (reference main.c:311-992, arena path):
 * *state is the xorshift64* state, advanced once.  logits_aligned: the
 * caller's logits are 32-byte aligned; nucleus_all: top-p keeps every token
 * (the reference's prefix-sum allocation failed). */
uint32_t or_sample_token(const float* logits, uint32_t V, float temperature, uint32_t top_k, float top_p,
                         int logits_aligned, int nucleus_all, uint64_t* state);
void or_add(const float* a, const float* b, float* out, uint32_t N);
void or_mul(const float* a, const float* b, float* out, uint32_t N);
void or_causal_mask(float* m, uint32_t n, uint32_t ld, float v);
/* Dot product in the order of q_matmul_f32_avx2's inner loop. */
float or_dot_f32(const float* a, const float* b, uint32_t K);
/* C[M x N] = A[M x K] . B[K x N] (row-major, dense). */
void or_matmul_f32(const float* A, const float* B, float* C, uint32_t M, uint32_t K, uint32_t N);

/* Decode attention for one token over cached positions 0..pos (inclusive).
 * q: [n_heads][head_dim] (already RoPE'd); kv_layer: [n_kv][max_seq][2][head_dim];
 * out: [n_heads][head_dim]. */
void or_attention_decode(const float* q, const float* kv_layer, float* out,
                         uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t max_seq, uint32_t pos);

/* Decode-step model description (device-independent, host pointers). */
typedef struct {
    uint32_t vocab, dim, hidden, n_layers, n_heads, n_kv_heads, max_seq;
    float rope_base, eps;
    const float* embd;         /* [vocab][dim] */
    const float* output_norm;  /* [dim] */
    const uint8_t* lm_head;    /* Q4_0 [vocab][dim] */
    const float* const* attn_norm; /* per layer [dim] */
    const uint8_t* const* wq;      /* Q4_0 [dim][dim] */
    const uint8_t* const* wk;      /* Q4_0 [kv_dim][dim] */
    const uint8_t* const* wv;
    const uint8_t* const* wo;      /* Q4_0 [dim][dim] */
    const float* const* ffn_norm;
    const uint8_t* const* w_gate;  /* Q4_0 [hidden][dim] */
    const uint8_t* const* w_up;
    const uint8_t* const* w_down;  /* Q4_0 [dim][hidden] */
    float* kv;                     /* [L][n_kv][max_seq][2][head_dim], updated */
} or_model;

/* One decode step: token at position pos; writes logits [vocab] and returns
 * the greedy token. */
uint32_t or_decode_step(const or_model* m, uint32_t token, uint32_t pos, float* logits);

/* Prefill GEMM through per-row GEMV: Y[T x M] = X[T x N] . W^T. */
void or_gemm_q4_rows(const uint8_t* W, uint32_t M, uint32_t N, const float* X,
                     uint32_t T, float* Y);

#ifdef __cplusplus
}
#endif

#endif
