// api_vec.cpp -- RMSNorm, RoPE, SiLU, softmax, add, mul and argmax entry
// points.  Host-pointer functions (qorus.h) reproduce the reference's
// validation order and codes, stage their arrays through HBM and return
// after the result is back on the host; qh_* functions (qorus_hip.h) take
// device pointers and enqueue on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>

#include "qh_kernels.hpp"
#include "qh_runtime.hpp"

namespace qh {

// Carves one staging slot into 256-byte aligned device arrays.
struct Stager {
    Device* d = nullptr;
    uint8_t* base = nullptr;
    size_t off = 0;
    static size_t round(size_t b) { return (b + 255) & ~(size_t)255; }
    q_error_code open(Device* dev, size_t total) {
        d = dev;
        void* p;
        QH_TRY_CODE(stage(dev, 1, total, &p));
        base = static_cast<uint8_t*>(p);
        off = 0;
        return Q_OK;
    }
    float* take(size_t n_floats) {
        float* p = reinterpret_cast<float*>(base + off);
        off += round(n_floats * 4);
        return p;
    }
    q_error_code put(float* dst, const float* src, size_t n) {
        if (n) QH_TRY(hipMemcpyAsync(dst, src, n * 4, hipMemcpyHostToDevice, d->stream));
        return Q_OK;
    }
    q_error_code get(float* dst, const float* src, size_t n) {
        if (n) QH_TRY(hipMemcpyAsync(dst, src, n * 4, hipMemcpyDeviceToHost, d->stream));
        QH_TRY(hipStreamSynchronize(d->stream));
        return Q_OK;
    }
};

static q_error_code validate_rmsnorm(const float* x, const float* w, const float* y, uint32_t N) {
    // reference src/ops/avx2/rmsnorm.c:22-31
    if (!x || !w || !y) return Q_ERR_INVALID_ARG;
    if (!aligned(x, 32) || !aligned(w, 32) || !aligned(y, 32)) return Q_ERR_MISALIGNED;
    if (N == 0 || N % 8 != 0) return Q_ERR_INVALID_SIZE;
    return Q_OK;
}

static q_error_code validate_rope(const float* x, const float* c, const float* s, const float* y, uint32_t N) {
    // reference src/ops/avx2/rope.c:32-43
    if (!x || !c || !s || !y) return Q_ERR_INVALID_ARG;
    if (!aligned(x, 32) || !aligned(c, 32) || !aligned(s, 32) || !aligned(y, 32)) return Q_ERR_MISALIGNED;
    if (N == 0 || N % 8 != 0 || N % 2 != 0) return Q_ERR_INVALID_SIZE;
    return Q_OK;
}

static q_error_code validate_silu(const float* x, const float* y, uint32_t N) {
    // reference src/ops/avx2/silu.c:24-64 (alignment only checked for N >= 8)
    if (!x || !y) return Q_ERR_INVALID_ARG;
    if (N == 0) return Q_ERR_INVALID_SIZE;
    if (N >= 8 && (!aligned(x, 32) || !aligned(y, 32))) return Q_ERR_MISALIGNED;
    return Q_OK;
}

static q_error_code validate_softmax(const float* x, const float* y, uint32_t N) {
    // reference src/ops/avx2/softmax.c:23-155 (alignment only checked for N >= 8)
    if (!x || !y) return Q_ERR_INVALID_ARG;
    if (N == 0) return Q_ERR_INVALID_SIZE;
    if (N >= 8 && (!aligned(x, 32) || !aligned(y, 32))) return Q_ERR_MISALIGNED;
    return Q_OK;
}

// reference src/ops/avx2/add_fp32.c:23-115 (mul_fp32.c:23-77 is identical).
static q_error_code validate_binary(const q_tensor* a, const q_tensor* b, const q_tensor* o, uint32_t* N) {
    if (!a || !b || !o) return Q_ERR_INVALID_ARG;
    if (!a->data || !b->data || !o->data) return Q_ERR_INVALID_ARG;
    if (!(a->ne[1] == 1 && a->ne[2] == 1 && a->ne[3] == 1)) return Q_ERR_INVALID_SIZE;
    if (!(b->ne[1] == 1 && b->ne[2] == 1 && b->ne[3] == 1)) return Q_ERR_INVALID_SIZE;
    if (!(o->ne[1] == 1 && o->ne[2] == 1 && o->ne[3] == 1)) return Q_ERR_INVALID_SIZE;
    const uint32_t n = a->ne[0];
    if (n != b->ne[0] || n != o->ne[0]) return Q_ERR_INVALID_SIZE;
    if (a->type != Q_F32 || b->type != Q_F32 || o->type != Q_F32) return Q_ERR_INVALID_DTYPE;
    const size_t row = (size_t)n * sizeof(float);
    if (a->nb[0] != row || b->nb[0] != row || o->nb[0] != row) return Q_ERR_INVALID_SIZE;
    if (!aligned(a->data, 32) || !aligned(b->data, 32) || !aligned(o->data, 32)) return Q_ERR_MISALIGNED;
    *N = n;
    return Q_OK;
}

static q_error_code host_binary(const q_tensor* a, const q_tensor* b, q_tensor* o, int op) {
    uint32_t N = 0;
    QH_TRY_CODE(validate_binary(a, b, o, &N));
    if (N == 0) return Q_OK;
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    QH_TRY_CODE(st.open(d, 3 * Stager::round((size_t)N * 4)));
    float* da = st.take(N);
    float* db = st.take(N);
    float* dout = st.take(N);
    QH_TRY_CODE(st.put(da, static_cast<const float*>(a->data), N));
    QH_TRY_CODE(st.put(db, static_cast<const float*>(b->data), N));
    QH_TRY(launch_binary(da, db, dout, N, op, d->stream));
    return st.get(static_cast<float*>(o->data), dout, N);
}

}  // namespace qh

using namespace qh;

extern "C" {

// Reference src/ops/avx2/matmul_fp32.c:57-300, validation in its order:
// NULL A/B/C/ctx -> INVALID_ARG; M, K or N zero, B->ne[0] != K, C->ne[0] !=
// M, C->ne[1] != N -> INVALID_SIZE; A->nb[0] % 32 == 0 with A->data not
// 32-byte aligned -> MISALIGNED (reported on stderr, as the reference
// does); any type != F32 -> INVALID_DTYPE; row strides below K (A), N (B)
// or the transposed B's column stride below K, or C's below N ->
// INVALID_SIZE; a non-transposed B then takes its N*K*4-byte transpose
// buffer from the arena (NULL -> ARENA_OOM).
q_error_code q_matmul_f32_avx2(const q_tensor* __restrict__ A, const q_tensor* __restrict__ B, q_tensor* C,
                               q_context* __restrict__ ctx) {
    if (!A || !B || !C || !ctx) return Q_ERR_INVALID_ARG;
    const uint32_t M = A->ne[0], K = A->ne[1], N = B->ne[1];
    if (M == 0 || K == 0 || N == 0) return Q_ERR_INVALID_SIZE;
    if (B->ne[0] != K || C->ne[0] != M || C->ne[1] != N) return Q_ERR_INVALID_SIZE;
    if (A->nb[0] % 32 == 0 && reinterpret_cast<uintptr_t>(A->data) % 32 != 0) {
        fprintf(stderr, "ERROR: q_matmul_f32_avx2: A->data not 32-byte aligned: %p\n", A->data);
        return Q_ERR_MISALIGNED;
    }
    if (A->type != Q_F32 || B->type != Q_F32 || C->type != Q_F32) return Q_ERR_INVALID_DTYPE;
    const size_t lda = A->nb[0] / sizeof(float), ldb = B->nb[0] / sizeof(float), ldc = C->nb[0] / sizeof(float);
    if (lda < K) return Q_ERR_INVALID_SIZE;
    const bool bt = B->nb[0] == sizeof(float) && B->ne[0] > 1 && B->nb[1] > sizeof(float);
    if (bt) {
        if (B->nb[1] / sizeof(float) < K) return Q_ERR_INVALID_SIZE;
    } else if (ldb < N) {
        return Q_ERR_INVALID_SIZE;
    }
    if (ldc < N) return Q_ERR_INVALID_SIZE;
    if (!bt && !q_arena_alloc(ctx, (size_t)N * K * sizeof(float))) return Q_ERR_ARENA_OOM;

    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    QH_TRY_CODE(st.open(d, Stager::round((size_t)M * K * 4) + Stager::round((size_t)K * N * 4) +
                               Stager::round((size_t)M * N * 4)));
    float* dA = st.take((size_t)M * K);
    float* dB = st.take((size_t)K * N);
    float* dC = st.take((size_t)M * N);
    hipStream_t s = d->stream;
    // Compact device copies of exactly the elements the reference reads.
    QH_TRY(hipMemcpy2DAsync(dA, (size_t)K * 4, A->data, lda * 4, (size_t)K * 4, M, hipMemcpyHostToDevice, s));
    if (bt)
        QH_TRY(hipMemcpyAsync(dB, B->data, (size_t)N * K * 4, hipMemcpyHostToDevice, s));
    else
        QH_TRY(hipMemcpy2DAsync(dB, (size_t)N * 4, B->data, ldb * 4, (size_t)N * 4, K, hipMemcpyHostToDevice, s));
    QH_TRY(launch_matmul_f32(dA, K, dB, bt ? K : N, bt, dC, N, M, N, K, s));
    QH_TRY(hipMemcpy2DAsync(C->data, ldc * 4, dC, (size_t)N * 4, (size_t)N * 4, M, hipMemcpyDeviceToHost, s));
    QH_TRY(hipStreamSynchronize(s));
    return Q_OK;
}

// Reference src/ops/avx2/causal_mask_fp32.c:16-138, validation in its
// order: NULL scores or data -> INVALID_ARG; ne[0] == 0 or ne[0] != ne[1] ->
// INVALID_SIZE; type != F32 -> INVALID_DTYPE; data not 32-byte aligned ->
// MISALIGNED; n == 1 -> OK (nothing above the diagonal); row stride
// nb[0]/4 < n -> INVALID_SIZE.  The n rows are staged through HBM and come
// back whole (only the strict upper triangle changes).
q_error_code q_causal_mask_f32_avx2(q_tensor* scores, float mask_value) {
    if (!scores || !scores->data) return Q_ERR_INVALID_ARG;
    const uint32_t n = scores->ne[0];
    if (n == 0 || n != scores->ne[1]) return Q_ERR_INVALID_SIZE;
    if (scores->type != Q_F32) return Q_ERR_INVALID_DTYPE;
    if (!aligned(scores->data, 32)) return Q_ERR_MISALIGNED;
    if (n == 1) return Q_OK;
    const size_t ld = scores->nb[0] / sizeof(float);
    if (ld < n) return Q_ERR_INVALID_SIZE;
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    QH_TRY_CODE(st.open(d, Stager::round((size_t)n * n * 4)));
    float* dm = st.take((size_t)n * n);
    hipStream_t s = d->stream;
    float* hm = static_cast<float*>(scores->data);
    QH_TRY(hipMemcpy2DAsync(dm, (size_t)n * 4, hm, ld * 4, (size_t)n * 4, n, hipMemcpyHostToDevice, s));
    QH_TRY(launch_causal_mask(dm, n, n, mask_value, s));
    QH_TRY(hipMemcpy2DAsync(hm, ld * 4, dm, (size_t)n * 4, (size_t)n * 4, n, hipMemcpyDeviceToHost, s));
    QH_TRY(hipStreamSynchronize(s));
    return Q_OK;
}

q_error_code qh_causal_mask_f32(float* scores, uint32_t n, uint32_t ld, float mask_value, qh_stream s) {
    if (!scores) return Q_ERR_INVALID_ARG;
    if (n == 0 || ld < n) return Q_ERR_INVALID_SIZE;
    if (n == 1) return Q_OK;
    if (!device_range(scores, ((size_t)(n - 1) * ld + n) * 4))
        return fail(hipErrorInvalidValue, "qh_causal_mask_f32: scores is not device memory of n rows");
    QH_TRY(launch_causal_mask(scores, n, ld, mask_value, (hipStream_t)s));
    return Q_OK;
}

q_error_code q_rmsnorm_f32_avx2(const float* __restrict__ x, const float* __restrict__ weight,
                                float* __restrict__ output, uint32_t N, float eps) {
    QH_TRY_CODE(validate_rmsnorm(x, weight, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    QH_TRY_CODE(st.open(d, 3 * Stager::round((size_t)N * 4)));
    float* dx = st.take(N);
    float* dw = st.take(N);
    float* dy = st.take(N);
    QH_TRY_CODE(st.put(dx, x, N));
    QH_TRY_CODE(st.put(dw, weight, N));
    QH_TRY(launch_rmsnorm(dx, dw, dy, N, eps, d->stream));
    return st.get(output, dy, N);
}

q_error_code q_rope_f32_avx2(const float* __restrict__ x, const float* __restrict__ cos,
                             const float* __restrict__ sin, float* __restrict__ output, uint32_t N) {
    QH_TRY_CODE(validate_rope(x, cos, sin, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    QH_TRY_CODE(st.open(d, 4 * Stager::round((size_t)N * 4)));
    float* dx = st.take(N);
    float* dc = st.take(N);
    float* ds = st.take(N);
    float* dy = st.take(N);
    QH_TRY_CODE(st.put(dx, x, N));
    QH_TRY_CODE(st.put(dc, cos, N));
    QH_TRY_CODE(st.put(ds, sin, N));
    QH_TRY(launch_rope(dx, dc, ds, dy, N, 1, d->stream));
    return st.get(output, dy, N);
}

q_error_code q_silu_f32_avx2(const float* __restrict__ x, float* __restrict__ output, uint32_t N) {
    QH_TRY_CODE(validate_silu(x, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    QH_TRY_CODE(st.open(d, 2 * Stager::round((size_t)N * 4)));
    float* dx = st.take(N);
    float* dy = st.take(N);
    QH_TRY_CODE(st.put(dx, x, N));
    QH_TRY(launch_silu(dx, nullptr, dy, N, d->stream));
    return st.get(output, dy, N);
}

q_error_code q_softmax_f32_avx2(const float* __restrict__ x, float* __restrict__ output, uint32_t N) {
    QH_TRY_CODE(validate_softmax(x, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    Stager st;
    const size_t wsb = softmax_exact_ws_bytes(N);
    QH_TRY_CODE(st.open(d, Stager::round((size_t)N * 4) + Stager::round(wsb)));
    float* dx = st.take(N);
    float* ws = st.take((wsb + 3) / 4);
    QH_TRY_CODE(st.put(dx, x, N));
    QH_TRY(launch_softmax_exact(dx, dx, N, ws, wsb, d->stream));
    return st.get(output, dx, N);
}

q_error_code q_add_f32_avx2(const q_tensor* a, const q_tensor* b, q_tensor* output) {
    return host_binary(a, b, output, 0);
}

q_error_code q_mul_f32_avx2(const q_tensor* a, const q_tensor* b, q_tensor* output) {
    return host_binary(a, b, output, 1);
}

// ---- device entry points ----

q_error_code qh_rmsnorm_f32(const float* x, const float* weight, float* output, uint32_t N, float eps,
                            qh_stream s) {
    QH_TRY_CODE(validate_rmsnorm(x, weight, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_rmsnorm(x, weight, output, N, eps, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_rope_f32(const float* x, const float* cos, const float* sin, float* output, uint32_t N,
                         uint32_t n_vec, qh_stream s) {
    QH_TRY_CODE(validate_rope(x, cos, sin, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_rope(x, cos, sin, output, N, n_vec, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_silu_f32(const float* x, float* output, uint32_t N, qh_stream s) {
    QH_TRY_CODE(validate_silu(x, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_silu(x, nullptr, output, N, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_silu_mul_f32(const float* gate, const float* up, float* output, uint32_t N, qh_stream s) {
    QH_TRY_CODE(validate_silu(gate, output, N));
    if (!up) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_silu(gate, up, output, N, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_softmax_f32(const float* x, float* output, uint32_t N, qh_stream s) {
    QH_TRY_CODE(validate_softmax(x, output, N));
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_softmax_exact(x, output, N, d->reduce_ws, kReduceWsBytes, (hipStream_t)s));
    return Q_OK;
}

size_t qh_softmax_workspace_bytes(uint32_t N) {
    const size_t a = softmax_workspace_bytes(N), b = softmax_exact_ws_bytes(N);
    return a > b ? a : b;
}
size_t qh_argmax_workspace_bytes(uint32_t N) { return argmax_workspace_bytes(N); }

q_error_code qh_softmax_f32_ws(const float* x, float* output, uint32_t N, void* workspace, qh_stream s) {
    QH_TRY_CODE(validate_softmax(x, output, N));
    if (!workspace) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_softmax_exact(x, output, N, workspace, softmax_exact_ws_bytes(N), (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_softmax_argmax_f32_ws(const float* x, float* output, uint32_t N, uint32_t* index_out,
                                      void* workspace, qh_stream s) {
    QH_TRY_CODE(validate_softmax(x, output, N));
    if (!index_out || !workspace) return Q_ERR_INVALID_ARG;
    if (x == output) return Q_ERR_ALIASING;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_softmax_argmax_ws(x, output, N, static_cast<float*>(workspace), index_out, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_add_f32(const float* a, const float* b, float* output, uint32_t N, qh_stream s) {
    if (!a || !b || !output) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_binary(a, b, output, N, 0, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_mul_f32(const float* a, const float* b, float* output, uint32_t N, qh_stream s) {
    if (!a || !b || !output) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_binary(a, b, output, N, 1, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_argmax_f32(const float* x, uint32_t N, uint32_t* index_out, qh_stream s) {
    if (!x || !index_out) return Q_ERR_INVALID_ARG;
    if (N == 0) return Q_ERR_INVALID_SIZE;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_argmax_ws(x, N, index_out, nullptr, nullptr, nullptr, 0, d->reduce_ws, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_argmax_f32_ws(const float* x, uint32_t N, uint32_t* index_out, void* workspace, qh_stream s) {
    if (!x || !index_out || !workspace) return Q_ERR_INVALID_ARG;
    if (N == 0) return Q_ERR_INVALID_SIZE;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_argmax_ws(x, N, index_out, nullptr, nullptr, nullptr, 0, static_cast<float*>(workspace),
                            (hipStream_t)s));
    return Q_OK;
}

}  // extern "C"
