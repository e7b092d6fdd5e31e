/*
 * qorus_oracle.c -- CPU ORACLE (test infrastructure only; never shipped,
 * never called by the product path) for the Qorus-IA quantized matrix path.
 *
 * Build: gcc -std=c11 -O3 -march=x86-64-v3 -ffp-contract=off (see Makefile).
 * -ffp-contract=off reproduces the reference's ISO-C build, where only the
 * explicit FMA intrinsics fuse; every fmaf() below stands for one of them.
 *
 * How each function is pinned (checked by tests/test_oracle_*.py):
 *   or_dequant_block   reference fixtures test_data/dequantize_test{1..4}
 *                      (tests/golden/), the adversarial block patterns of
 *                      tests/test_dequantize_adversarial.c, the closed form
 *                      (q-8)*s, and bit-equality with oracle/_ref.
 *   or_gemv_q4         bit-equality with oracle/_ref (the reference's own
 *                      q_gemv_q4_f32_avx2 compiled from its sources), fp64
 *                      closed form, all blocks%4 tails on brute-force sizes.
 *   or_rmsnorm         closed form x/sqrt(mean+eps)*w in fp64; tolerance vs
 *                      oracle/_ref (rsqrtps seed is CPU-specific, so bits are
 *                      not portable: parity is tolerance-only by nature).
 *   or_rope            bit-equality with oracle/_ref; rotation invariants.
 *   or_rope_tables     bit-equality, every position 0..2047 and every
 *                      pair, with the cache the reference's own
 *                      llama_build_graph builds in oracle/_ref (head_dim
 *                      128/base 500000 and 64/10000); each entry within 1 ulp
 *                      of float64 cos/sin along the builder's float32 chain
 *                      freq_i = base^(-2i/hd), theta = freq_i * pos.
 *   or_exp_approx      bit-equality with oracle/_ref's softmax/silu outputs;
 *                      polynomial special cases (x<-10 -> 0, x>10 -> 22026).
 *   or_silu/softmax    bit-equality with oracle/_ref on the vector part; the
 *                      N%8 tails use libm expf (unpinned libm boundary).
 *   or_argmax          brute force + first-index-on-ties cases.
 *   or_sample_token    token-for-token equality with oracle/_ref's own
 *                      q_sample_token (reference src/main.c compiled from its
 *                      sources, arena path, a fresh RNG state per library
 *                      copy) on inputs whose top-k/top-p cut has no ties, for
 *                      temperatures, top-k, top-p and aligned/unaligned
 *                      logits; the reference's own property tests
 *                      (tests/test_main.c).  Its two rules for what the
 *                      reference leaves to its sort internals or to unwritten
 *                      memory (ties at a cut keep lower indices; no filter
 *                      keeps every token) have no reference fixture.
 *   or_add/mul         bit-equality with oracle/_ref.
 *   or_causal_mask     bit-equality with oracle/_ref's q_causal_mask_f32_avx2
 *                      (every seq_len 1..70 and 255/256/257, row stride n and
 *                      n + 8, NaN payloads below the diagonal and in the
 *                      stride padding); brute-force index rule.
 *   or_dot_f32/matmul  bit-equality with oracle/_ref's q_matmul_f32_avx2.
 *   or_attention_decode  composition of the above; fp64 textbook attention
 *                      (with the polynomial exp) within tolerance.
 *   or_decode_step     no reference fixture exists (the reference forward
 *                      never reads its KV cache and its dummy model holds
 *                      FP32 bytes in Q4 slots).  Pinned through its parts and,
 *                      as a composition, against a float64 restatement
 *                      written from the Llama-3 equations (tests/llama_f64.py):
 *                      same greedy token, logits within 1e-4 of the largest
 *                      |logit| and the same cache row, on 2-layer models with
 *                      GQA groups 1/2/4 at pos 0 and at pos 13 over a random
 *                      cache; planted composition mistakes (GQA mapping,
 *                      RoPE position or pairing, residual, norm weight) fail
 *                      that comparison.
 */
#include "qorus_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Q4_0 dequantization.  Reference src/ops/avx2/dequantize.c:18-73:
 * off = -8*s (one multiply), out[e] = fma((float)q_e, s, off), element e in
 * byte e>>1, low nibble for even e. */
static inline float blk_scale(const uint8_t* blk) {
    float s;
    memcpy(&s, blk + 16, 4);
    return s;
}

static inline uint32_t blk_nib(const uint8_t* blk, uint32_t e) {
    const uint8_t b = blk[e >> 1];
    return (e & 1u) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0x0F);
}

void or_dequant_block(const uint8_t* blk, float out[32]) {
    const float s = blk_scale(blk);
    const float off = -8.0f * s;
    for (uint32_t e = 0; e < 32; e++) out[e] = fmaf((float)blk_nib(blk, e), s, off);
}

void or_dequant_blocks(const uint8_t* blks, uint64_t n_blocks, float* out) {
    for (uint64_t b = 0; b < n_blocks; b++) or_dequant_block(blks + b * 20, out + b * 32);
}

/* ------------------------------------------------------------------------ */
/* Horizontal reductions of an 8-lane vector in the reference's shuffle order
 * (src/ops/avx2/avx_math.h:64-85, matmul.c:252-265): ((v0+v4)+(v1+v5)) +
 * ((v2+v6)+(v3+v7)). */
static inline float hsum8(const float v[8]) {
    const float t0 = v[0] + v[4], t1 = v[1] + v[5], t2 = v[2] + v[6], t3 = v[3] + v[7];
    return (t0 + t1) + (t2 + t3);
}

/* maxps(a,b) returns b unless a > b (NaN-propagation as on x86). */
static inline float maxps(float a, float b) { return a > b ? a : b; }
static inline float minps(float a, float b) { return a < b ? a : b; }

static inline float hmax8(const float v[8]) {
    const float t0 = maxps(v[0], v[4]), t1 = maxps(v[1], v[5]);
    const float t2 = maxps(v[2], v[6]), t3 = maxps(v[3], v[7]);
    return maxps(maxps(t0, t1), maxps(t2, t3));
}

/* ------------------------------------------------------------------------ */
/* GEMV.  Reference src/ops/avx2/matmul.c:43-96 (per block) and :199-266
 * (row loop): four 8-lane accumulators; block b = 4g+u feeds acc[u]; the
 * 0-3 tail blocks feed acc[0..2]; element e = 8k+l of a block feeds lane l;
 * w = fma(q, s, -8s); acc = fma(w, x, acc). */
static void gemv_row(const uint8_t* row, uint32_t nblk, const float* x, float* y) {
    float acc[4][8];
    memset(acc, 0, sizeof(acc));
    const uint32_t groups = nblk / 4;
    for (uint32_t b = 0; b < nblk; b++) {
        const uint32_t u = (b < groups * 4) ? (b & 3u) : (b - groups * 4);
        const uint8_t* blk = row + (size_t)b * 20;
        const float s = blk_scale(blk);
        const float off = -8.0f * s;
        const float* xb = x + (size_t)b * 32;
        for (uint32_t k = 0; k < 4; k++) {
            for (uint32_t l = 0; l < 8; l++) {
                const uint32_t e = 8 * k + l;
                const float w = fmaf((float)blk_nib(blk, e), s, off);
                acc[u][l] = fmaf(w, xb[e], acc[u][l]);
            }
        }
    }
    float sl[8];
    for (uint32_t l = 0; l < 8; l++) sl[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    *y = hsum8(sl);
}

/* Threads for the row loops of the GEMV and the heads of the attention (1 by
 * default).  Each row / head is computed by one thread in the order above,
 * so the results are the same bits for any count; more threads only make
 * long oracle runs (deep models, 512-token prompts) finish sooner. */
static int g_threads = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

void or_gemv_q4_rows(const uint8_t* W, uint32_t r0, uint32_t r1, uint32_t N,
                     const float* x, float* y) {
    const uint32_t nblk = N / 32;
    const size_t row_bytes = (size_t)nblk * 20;
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && r1 - r0 >= 256)
    for (uint32_t i = r0; i < r1; i++) gemv_row(W + (size_t)i * row_bytes, nblk, x, &y[i]);
}

void or_gemv_q4(const uint8_t* W, uint32_t M, uint32_t N, const float* x, float* y) {
    or_gemv_q4_rows(W, 0, M, N, x, y);
}

void or_gemv_q4_f64(const uint8_t* W, uint32_t M, uint32_t N, const float* x,
                    double* y64, double* cond) {
    const uint32_t nblk = N / 32;
    const size_t row_bytes = (size_t)nblk * 20;
    for (uint32_t i = 0; i < M; i++) {
        const uint8_t* row = W + (size_t)i * row_bytes;
        double acc = 0.0, c = 0.0;
        for (uint32_t b = 0; b < nblk; b++) {
            const uint8_t* blk = row + (size_t)b * 20;
            const double s = (double)blk_scale(blk);
            for (uint32_t e = 0; e < 32; e++) {
                const double p = ((double)blk_nib(blk, e) - 8.0) * s * (double)x[(size_t)b * 32 + e];
                acc += p;
                c += fabs(p);
            }
        }
        y64[i] = acc;
        if (cond) cond[i] = c;
    }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm.  Reference src/ops/avx2/rmsnorm.c:33-89: lane sums of x*x (mul
 * then add), hsum, mean = sum/(float)N, a = mean + eps, r = rsqrt(a) refined
 * once by Newton: r' = (r * (3 - a*(r*r))) * 0.5, y = (x*r')*w.  The
 * reference seed is the CPU's rsqrtps estimate; the oracle seeds with the
 * correctly rounded 1/sqrtf(a). */
void or_rmsnorm(const float* x, const float* w, float* y, uint32_t N, float eps) {
    float ss[8] = {0};
    for (uint32_t i = 0; i < N / 8; i++)
        for (uint32_t l = 0; l < 8; l++) {
            const float v = x[8 * i + l];
            const float sq = v * v;
            ss[l] = ss[l] + sq;
        }
    const float sum = hsum8(ss);
    const float mean = sum / (float)N;
    const float a = mean + eps;
    const float r0 = 1.0f / sqrtf(a);
    const float r = (r0 * (3.0f - a * (r0 * r0))) * 0.5f;
    for (uint32_t i = 0; i < N; i++) {
        const float n = x[i] * r;
        y[i] = n * w[i];
    }
}

/* ------------------------------------------------------------------------ */
/* RoPE.  Reference src/ops/avx2/rope.c:63-106: pair (x0,x1) = (x[2p],x[2p+1])
 * with c = cos[2p], s = sin[2p]: y0 = x0*c - x1*s, y1 = x1*c + x0*s, each
 * product rounded before the add/sub. */
void or_rope(const float* x, const float* cos_t, const float* sin_t, float* y, uint32_t N) {
    for (uint32_t i = 0; i < N; i += 2) {
        const float x0 = x[i], x1 = x[i + 1];
        const float c = cos_t[i], s = sin_t[i];
        const float a0 = x0 * c, b0 = x1 * s;
        const float a1 = x1 * c, b1 = x0 * s;
        y[i] = a0 - b0;
        y[i + 1] = a1 + b1;
    }
}

/* Tables.  Reference src/models/model.c:633-659: freq_i =
 * powf(base, (-2.0f*(float)i)/(float)head_dim); theta = freq_i*(float)pos;
 * cos/sin duplicated per pair. */
void or_rope_tables(float base, uint32_t head_dim, uint32_t pos, float* cos_t, float* sin_t) {
    for (uint32_t i = 0; i < head_dim / 2; i++) {
        const float fe = -2.0f * (float)i / (float)head_dim;
        const float freq = powf(base, fe);
        const float th = freq * (float)pos;
        const float c = cosf(th), s = sinf(th);
        cos_t[2 * i] = c;
        cos_t[2 * i + 1] = c;
        sin_t[2 * i] = s;
        sin_t[2 * i + 1] = s;
    }
}

/* ------------------------------------------------------------------------ */
/* Polynomial exp.  Reference src/ops/avx2/avx_math.h:10-61: flags on the
 * unclamped x (ordered compares), clamp with minps/maxps to [-5, 5], degree-5
 * Horner in FMA, max(r, 0), x < -10 -> 0, x > 10 -> 22026. */
float or_exp_approx(float x) {
    const int very_neg = x < -10.0f;
    const int very_pos = x > 10.0f;
    float t = minps(x, 5.0f);
    t = maxps(t, -5.0f);
    float r = 0.00833333f;
    r = fmaf(r, t, 0.04166667f);
    r = fmaf(r, t, 0.16666667f);
    r = fmaf(r, t, 0.5f);
    r = fmaf(r, t, 1.0f);
    r = fmaf(r, t, 1.0f);
    r = maxps(r, 0.0f);
    if (very_neg) r = 0.0f;
    if (very_pos) r = 22026.0f;
    return r;
}

/* SiLU.  Reference src/ops/avx2/silu.c:44-91: for N >= 8 the first N&~7
 * elements use y = x * (1 / (1 + exp_approx(-x))); the rest, and every
 * element when N < 8, use libm expf. */
void or_silu(const float* x, float* y, uint32_t N) {
    const uint32_t nv = (N >= 8) ? (N & ~7u) : 0;
    for (uint32_t i = 0; i < nv; i++) {
        const float e = or_exp_approx(-x[i]);
        const float d = 1.0f + e;
        const float sg = 1.0f / d;
        y[i] = x[i] * sg;
    }
    for (uint32_t i = nv; i < N; i++) {
        const float sg = 1.0f / (1.0f + expf(-x[i]));
        y[i] = x[i] * sg;
    }
}

/* Softmax.  Reference src/ops/avx2/softmax.c:30-213.  N >= 8: 8-lane max
 * (maxps), hmax, scalar tail max (strict >), e = exp_approx(x - max) with
 * lane sums, hsum, tail e = expf(x - max) summed sequentially after the
 * hsum, inv = 1/sum, y = e*inv.  N < 8: libm expf, sequential sum, y = e/sum. */
void or_softmax(const float* x, float* y, uint32_t N) {
    if (N == 0) return;
    if (N < 8) {
        float mx = x[0];
        for (uint32_t i = 1; i < N; i++)
            if (x[i] > mx) mx = x[i];
        float sum = 0.0f;
        for (uint32_t i = 0; i < N; i++) {
            const float e = expf(x[i] - mx);
            y[i] = e;
            sum += e;
        }
        for (uint32_t i = 0; i < N; i++) y[i] = y[i] / sum;
        return;
    }
    const uint32_t nv = N & ~7u;
    float lm[8];
    for (uint32_t l = 0; l < 8; l++) lm[l] = -INFINITY;
    for (uint32_t i = 0; i < nv; i += 8)
        for (uint32_t l = 0; l < 8; l++) lm[l] = maxps(lm[l], x[i + l]);
    float mx = hmax8(lm);
    for (uint32_t i = nv; i < N; i++)
        if (x[i] > mx) mx = x[i];
    float ls[8] = {0};
    for (uint32_t i = 0; i < nv; i += 8)
        for (uint32_t l = 0; l < 8; l++) {
            const float d = x[i + l] - mx;
            const float e = or_exp_approx(d);
            ls[l] = ls[l] + e;
            y[i + l] = e;
        }
    float sum = hsum8(ls);
    for (uint32_t i = nv; i < N; i++) {
        const float e = expf(x[i] - mx);
        y[i] = e;
        sum += e;
    }
    const float inv = 1.0f / sum;
    for (uint32_t i = 0; i < N; i++) y[i] = y[i] * inv;
}

/* Sampling.  Reference src/main.c:311-992 (q_sample_token with an arena:
 * compute_softmax_with_temp, apply_top_k, apply_top_p with
 * find_nucleus_size_optimized_soa's binary search over the full prefix
 * sums, the xorshift64* draw, sample_from_distribution), restated with
 * (p desc, index asc) ordering where the reference's quickselect/quicksort
 * leave equal probabilities in an order of their own, and every token valid
 * when neither filter is on (the reference reads an unwritten mask). */
typedef struct {
    uint32_t key, idx;
} or_kv;

static int or_kv_desc(const void* a, const void* b) {
    const or_kv* x = (const or_kv*)a;
    const or_kv* y = (const or_kv*)b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx ? 1 : 0);
}

static void or_sort_desc(const float* p, uint32_t V, or_kv* kv) {
    for (uint32_t i = 0; i < V; i++) {
        uint32_t b;
        memcpy(&b, &p[i], 4);
        kv[i].key = b == 0x80000000u ? 0u : b;
        kv[i].idx = i;
    }
    qsort(kv, V, sizeof(or_kv), or_kv_desc);
}

uint32_t or_sample_token(const float* logits, uint32_t V, float temperature, uint32_t top_k, float top_p,
                         int logits_aligned, int nucleus_all, uint64_t* state) {
    float* sc = (float*)malloc((size_t)V * sizeof(float));
    float* p = (float*)malloc((size_t)V * sizeof(float));
    float* cs = (float*)malloc((size_t)V * sizeof(float));
    uint8_t* m = (uint8_t*)malloc(V);
    or_kv* kv = (or_kv*)malloc((size_t)V * sizeof(or_kv));
    /* temperature: 8-wide part times 1/T when the logits are aligned,
     * the rest divided (main.c:338-365) */
    const float inv = 1.0f / temperature;
    const uint32_t n_mul = (V >= 8 && logits_aligned) ? (V & ~7u) : 0u;
    for (uint32_t i = 0; i < V; i++) sc[i] = i < n_mul ? logits[i] * inv : logits[i] / temperature;
    /* softmax: q_softmax_f32_avx2 for V >= 8 (main.c:371-385), else the
     * sampler's scalar fallback (main.c:389-424) */
    if (V >= 8) {
        or_softmax(sc, p, V);
    } else {
        float mx = sc[0];
        for (uint32_t i = 1; i < V; i++)
            if (sc[i] > mx) mx = sc[i];
        float sum = 0.0f;
        for (uint32_t i = 0; i < V; i++) {
            p[i] = expf(sc[i] - mx);
            sum += p[i];
        }
        if (sum > 0.0f) {
            const float is = 1.0f / sum;
            for (uint32_t i = 0; i < V; i++) p[i] *= is;
        } else {
            const float u = 1.0f / (float)V;
            for (uint32_t i = 0; i < V; i++) p[i] = u;
        }
    }
    int mask_set = 0;
    /* top-k (main.c:431-521) */
    if (top_k > 0) {
        if (top_k >= V) {
            memset(m, 1, V);
        } else {
            or_sort_desc(p, V, kv);
            memset(m, 0, V);
            float sum = 0.0f;
            for (uint32_t j = 0; j < top_k; j++) {
                m[kv[j].idx] = 1;
                sum += p[kv[j].idx];
            }
            if (sum > 0.0f)
                for (uint32_t i = 0; i < V; i++) p[i] = m[i] ? p[i] / sum : 0.0f;
        }
        mask_set = 1;
    }
    /* top-p (main.c:720-808, 525-597) */
    if (top_p > 0.0f) {
        if (top_p >= 1.0f) {
            memset(m, 1, V);
        } else {
            or_sort_desc(p, V, kv);
            uint32_t best = V;
            if (!nucleus_all) {
                cs[0] = p[kv[0].idx];
                for (uint32_t j = 1; j < V; j++) cs[j] = cs[j - 1] + p[kv[j].idx];
                uint32_t left = 1, right = V;
                while (left <= right) {
                    const uint32_t mid = left + (right - left) / 2;
                    if (cs[mid - 1] >= top_p) {
                        best = mid;
                        right = mid - 1;
                    } else {
                        left = mid + 1;
                    }
                }
            }
            memset(m, 0, V);
            float sum = 0.0f;
            for (uint32_t j = 0; j < best; j++) {
                m[kv[j].idx] = 1;
                sum += p[kv[j].idx];
            }
            if (sum > 0.0f)
                for (uint32_t i = 0; i < V; i++) p[i] = m[i] ? p[i] / sum : 0.0f;
        }
        mask_set = 1;
    }
    if (!mask_set) memset(m, 1, V);
    /* xorshift64* draw (main.c:949-968) */
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    const uint32_t u32 = (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
    const float r = (float)(u32 >> 8) / 16777216.0f;
    /* CDF walk over valid tokens in index order (main.c:811-849) */
    uint32_t tok = V - 1;
    int found = 0;
    float c = 0.0f;
    for (uint32_t i = 0; i < V && !found; i++)
        if (m[i]) {
            c += p[i];
            if (r < c) {
                tok = i;
                found = 1;
            }
        }
    if (!found)
        for (uint32_t i = V; i > 0; i--)
            if (m[i - 1]) {
                tok = i - 1;
                break;
            }
    free(sc);
    free(p);
    free(cs);
    free(m);
    free(kv);
    return tok;
}

/* Greedy argmax.  Reference src/main.c:870-881: first index, strict >. */
uint32_t or_argmax(const float* x, uint32_t N) {
    uint32_t idx = 0;
    float mx = x[0];
    for (uint32_t i = 1; i < N; i++)
        if (x[i] > mx) {
            mx = x[i];
            idx = i;
        }
    return idx;
}

/* Reference src/ops/avx2/add_fp32.c:127-161 and mul_fp32.c:89-123. */
void or_add(const float* a, const float* b, float* out, uint32_t N) {
    for (uint32_t i = 0; i < N; i++) out[i] = a[i] + b[i];
}

void or_mul(const float* a, const float* b, float* out, uint32_t N) {
    for (uint32_t i = 0; i < N; i++) out[i] = a[i] * b[i];
}

/* Reference src/ops/avx2/causal_mask_fp32.c:53-135: in row i of the n x n
 * matrix (row stride ld floats) every column j > i becomes v; the blend of
 * the boundary block selects by index (j > i), so the other elements keep
 * their bits, NaN payloads included; columns n .. ld-1 are not touched. */
void or_causal_mask(float* m, uint32_t n, uint32_t ld, float v) {
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t j = i + 1; j < n; j++) m[(size_t)i * ld + j] = v;
}

/* ------------------------------------------------------------------------ */
/* FP32 dot in the order of reference src/ops/avx2/matmul_fp32.c:339-453:
 * for K&~31 elements four 8-lane FMA accumulators (element k feeds
 * acc[(k%32)/8] lane k%8), lanewise (a0+a1)+(a2+a3), hsum; then the scalar
 * tail dot += a*b (separate multiply and add). */
float or_dot_f32(const float* a, const float* b, uint32_t K) {
    float dot = 0.0f;
    const uint32_t kv = K & ~31u;
    if (kv > 0) {
        float acc[4][8];
        memset(acc, 0, sizeof(acc));
        for (uint32_t k = 0; k < kv; k += 32)
            for (uint32_t c = 0; c < 4; c++)
                for (uint32_t l = 0; l < 8; l++)
                    acc[c][l] = fmaf(a[k + 8 * c + l], b[k + 8 * c + l], acc[c][l]);
        float sl[8];
        for (uint32_t l = 0; l < 8; l++) sl[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
        dot = hsum8(sl);
    }
    for (uint32_t k = kv; k < K; k++) {
        const float p = a[k] * b[k];
        dot = dot + p;
    }
    return dot;
}

void or_matmul_f32(const float* A, const float* B, float* C, uint32_t M, uint32_t K, uint32_t N) {
    float* bt = (float*)malloc((size_t)K * N * sizeof(float));
    for (uint32_t k = 0; k < K; k++)
        for (uint32_t j = 0; j < N; j++) bt[(size_t)j * K + k] = B[(size_t)k * N + j];
    for (uint32_t i = 0; i < M; i++)
        for (uint32_t j = 0; j < N; j++)
            C[(size_t)i * N + j] = or_dot_f32(A + (size_t)i * K, bt + (size_t)j * K, K);
    free(bt);
}

/* ------------------------------------------------------------------------ */
/* Decode attention over the cache (the reference composition of
 * src/models/model.c:1340-1440 -- QK^T by q_matmul_f32, separate multiply by
 * 1/sqrtf(head_dim), row softmax, P.V by q_matmul_f32 -- applied to keys
 * 0..pos read from the cache laid out as in get_kv_cache_ptr,
 * model.c:700-740: [kv_head][pos][K|V][head_dim]). */
void or_attention_decode(const float* q, const float* kv_layer, float* out,
                         uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t max_seq, uint32_t pos) {
    const uint32_t S = pos + 1;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t pos_stride = 2 * (size_t)head_dim;
    const size_t head_stride = (size_t)max_seq * pos_stride;
#pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
        float* sc = (float*)malloc((size_t)S * sizeof(float));
        float* vt = (float*)malloc((size_t)S * sizeof(float));
#pragma omp for schedule(static)
        for (uint32_t h = 0; h < n_heads; h++) {
            const uint32_t kvh = h / (n_heads / n_kv_heads);
            const float* base = kv_layer + (size_t)kvh * head_stride;
            const float* qh = q + (size_t)h * head_dim;
            for (uint32_t j = 0; j < S; j++) {
                const float d = or_dot_f32(qh, base + (size_t)j * pos_stride, head_dim);
                sc[j] = d * scale;
            }
            or_softmax(sc, sc, S);
            for (uint32_t d = 0; d < head_dim; d++) {
                for (uint32_t j = 0; j < S; j++) vt[j] = base[(size_t)j * pos_stride + head_dim + d];
                out[(size_t)h * head_dim + d] = or_dot_f32(sc, vt, S);
            }
        }
        free(sc);
        free(vt);
    }
}

/* ------------------------------------------------------------------------ */
/* One decode step with the corrected composition of reference
 * src/models/model.c:1568-1850 (layer, attention, MLP, final norm, LM head)
 * and src/main.c:870-881 (argmax): [out,in] matrix shapes, attention over
 * the cache, Q4_0 LM head. */
uint32_t or_decode_step(const or_model* m, uint32_t token, uint32_t pos, float* logits) {
    const uint32_t dim = m->dim, hid = m->hidden, hd = dim / m->n_heads;
    const uint32_t kvd = m->n_kv_heads * hd;
    float* x = (float*)malloc(dim * sizeof(float));
    float* h = (float*)malloc(dim * sizeof(float));
    float* q = (float*)malloc(dim * sizeof(float));
    float* qr = (float*)malloc(dim * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* o = (float*)malloc(dim * sizeof(float));
    float* a = (float*)malloc(dim * sizeof(float));
    float* x1 = (float*)malloc(dim * sizeof(float));
    float* g = (float*)malloc(hid * sizeof(float));
    float* u = (float*)malloc(hid * sizeof(float));
    float* gs = (float*)malloc(hid * sizeof(float));
    float* mm = (float*)malloc(hid * sizeof(float));
    float* cs = (float*)malloc(hd * sizeof(float));
    float* sn = (float*)malloc(hd * sizeof(float));

    memcpy(x, m->embd + (size_t)token * dim, dim * sizeof(float));
    or_rope_tables(m->rope_base, hd, pos, cs, sn);
    const size_t layer_kv = (size_t)m->n_kv_heads * m->max_seq * 2 * hd;
    for (uint32_t l = 0; l < m->n_layers; l++) {
        float* kvl = m->kv + (size_t)l * layer_kv;
        or_rmsnorm(x, m->attn_norm[l], h, dim, m->eps);
        or_gemv_q4(m->wq[l], dim, dim, h, q);
        or_gemv_q4(m->wk[l], kvd, dim, h, k);
        or_gemv_q4(m->wv[l], kvd, dim, h, v);
        for (uint32_t hh = 0; hh < m->n_heads; hh++) or_rope(q + hh * hd, cs, sn, qr + hh * hd, hd);
        for (uint32_t kh = 0; kh < m->n_kv_heads; kh++) {
            float* dst = kvl + ((size_t)kh * m->max_seq + pos) * 2 * hd;
            or_rope(k + kh * hd, cs, sn, dst, hd);
            memcpy(dst + hd, v + kh * hd, hd * sizeof(float));
        }
        or_attention_decode(qr, kvl, o, m->n_heads, m->n_kv_heads, hd, m->max_seq, pos);
        or_gemv_q4(m->wo[l], dim, dim, o, a);
        or_add(x, a, x1, dim);
        or_rmsnorm(x1, m->ffn_norm[l], h, dim, m->eps);
        or_gemv_q4(m->w_gate[l], hid, dim, h, g);
        or_gemv_q4(m->w_up[l], hid, dim, h, u);
        or_silu(g, gs, hid);
        or_mul(gs, u, mm, hid);
        or_gemv_q4(m->w_down[l], dim, hid, mm, a);
        or_add(x1, a, x, dim);
    }
    uint32_t tok = 0;
    if (logits) {  /* NULL: the cache rows only (a prompt's earlier tokens) */
        or_rmsnorm(x, m->output_norm, h, dim, m->eps);
        or_gemv_q4(m->lm_head, m->vocab, dim, h, logits);
        tok = or_argmax(logits, m->vocab);
    }
    free(x); free(h); free(q); free(qr); free(k); free(v); free(o); free(a);
    free(x1); free(g); free(u); free(gs); free(mm); free(cs); free(sn);
    return tok;
}

/* Prefill projection as the reference runs it: one GEMV per token row
 * (src/models/model.c:1120-1131, 1485-1512, 1555-1561). */
void or_gemm_q4_rows(const uint8_t* W, uint32_t M, uint32_t N, const float* X,
                     uint32_t T, float* Y) {
    for (uint32_t t = 0; t < T; t++) or_gemv_q4(W, M, N, X + (size_t)t * N, Y + (size_t)t * M);
}
