// api_q4.cpp -- Q4_0 dequantization and GEMV entry points.
//
// Host-pointer entry points (qorus.h) keep the reference's signature,
// validation order and return codes; device entry points (qorus_hip.h) share
// the same validation and enqueue on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>

#include "qh_kernels.hpp"
#include "qh_runtime.hpp"

namespace qh {

// Validation of reference src/ops/avx2/matmul.c:104-197, in its order:
// NULL W/x/y -> INVALID_ARG; x or y not 32-byte aligned -> MISALIGNED;
// x == y -> ALIASING; M == 0, N == 0, N % 32 -> INVALID_SIZE; type !=
// Q4_0 -> INVALID_DTYPE; N/32 > UINT32_MAX/M -> OVERFLOW; nb[0] != N/32*20
// -> INVALID_ARG.  Then, for the device kernel: W->data NULL -> INVALID_ARG
// and W->data not 4-byte aligned -> MISALIGNED (the reference reads any
// address; the GPU loads are dword-granular).
q_error_code validate_gemv(const q_tensor* W, const float* x, const float* y) {
    if (!W || !x || !y) return Q_ERR_INVALID_ARG;
    if (!aligned(x, 32) || !aligned(y, 32)) return Q_ERR_MISALIGNED;
    if (x == y) return Q_ERR_ALIASING;
    const uint32_t M = W->ne[0], N = W->ne[1];
    if (M == 0 || N == 0 || N % 32 != 0) return Q_ERR_INVALID_SIZE;
    if (W->type != Q_Q4_0) return Q_ERR_INVALID_DTYPE;
    const uint32_t bpr = N / 32;
    if (bpr > UINT32_MAX / M) return Q_ERR_OVERFLOW;
    if (W->nb[0] != (size_t)bpr * sizeof(q_block_q4_0)) return Q_ERR_INVALID_ARG;
    if (!W->data) return Q_ERR_INVALID_ARG;
    if (!aligned(W->data, 4)) return Q_ERR_MISALIGNED;
    return Q_OK;
}

// The library's GEMV digit workspace (allocated once with the device state)
// for device calls that pass none: inputs up to kLibGemvMaxN wide.  Calls
// that overlap on one device share it and race.
static q_error_code library_workspace(Device* d, uint32_t N, void** out) {
    if (N > kLibGemvMaxN)
        return fail_code(Q_ERR_INVALID_SIZE, "GEMV input wider than the library workspace: pass a workspace");
    *out = d->gemv_ws;
    return Q_OK;
}

static q_error_code gemv_device(const q_tensor* W, const void* wdev, const float* x, const float* res,
                                float* y, void* ws, hipStream_t s) {
    const uint32_t M = W->ne[0], N = W->ne[1];
    GemvSeg seg{static_cast<const uint8_t*>(wdev), y, res, M};
    QH_TRY(launch_gemv_f32(&seg, 1, N, x, static_cast<uint4*>(ws), s));
    return Q_OK;
}

// Workspace is only used by inputs wider than the in-kernel conversion.
static bool needs_workspace(uint32_t N) { return N / 32 > kGemvF32MaxBlk; }

}  // namespace qh

using namespace qh;

extern "C" {

size_t qh_gemv_workspace_bytes(uint32_t N) { return xd_bytes((N + 31) / 32); }

q_error_code qh_dequantize_q4_0(const void* blocks, float* out, uint64_t n_blocks, qh_stream s) {
    if (!blocks || !out) return Q_ERR_INVALID_ARG;
    if (!aligned(blocks, 4) || !aligned(out, 16)) return Q_ERR_MISALIGNED;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_dequant(static_cast<const uint8_t*>(blocks), out, n_blocks, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_gemv_q4_f32(const q_tensor* W, const float* x, float* y, void* workspace, qh_stream s) {
    QH_TRY_CODE(validate_gemv(W, x, y));
    Device* d;
    QH_TRY_CODE(device(&d));
    if (!workspace && needs_workspace(W->ne[1])) QH_TRY_CODE(library_workspace(d, W->ne[1], &workspace));
    return gemv_device(W, W->data, x, nullptr, y, workspace, (hipStream_t)s);
}

q_error_code qh_gemv_q4_f32_add(const q_tensor* W, const float* x, const float* residual, float* y,
                                void* workspace, qh_stream s) {
    QH_TRY_CODE(validate_gemv(W, x, y));
    if (!residual) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    if (!workspace && needs_workspace(W->ne[1])) QH_TRY_CODE(library_workspace(d, W->ne[1], &workspace));
    return gemv_device(W, W->data, x, residual, y, workspace, (hipStream_t)s);
}

q_error_code qh_gemv_prepare(const float* x, uint32_t N, void* workspace, qh_stream s) {
    if (!x || !workspace) return Q_ERR_INVALID_ARG;
    if (!aligned(x, 32)) return Q_ERR_MISALIGNED;
    if (N == 0 || N % 32 != 0) return Q_ERR_INVALID_SIZE;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_xprep(x, N, nullptr, 0.0f, nullptr, static_cast<uint4*>(workspace), (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_gemv_q4_f32_prepared(const q_tensor* const* Ws, const float* const* residuals,
                                     float* const* ys, uint32_t n, const void* workspace, qh_stream s) {
    if (!Ws || !ys || !workspace) return Q_ERR_INVALID_ARG;
    if (n < 1 || n > 4) return Q_ERR_INVALID_SIZE;
    GemvSeg segs[4];
    for (uint32_t i = 0; i < n; ++i) {
        const q_tensor* W = Ws[i];
        if (!W || !ys[i]) return Q_ERR_INVALID_ARG;
        if (!aligned(ys[i], 32)) return Q_ERR_MISALIGNED;
        const uint32_t M = W->ne[0], N = W->ne[1];
        if (M == 0 || N == 0 || N % 32 != 0 || N != Ws[0]->ne[1]) return Q_ERR_INVALID_SIZE;
        if (W->type != Q_Q4_0) return Q_ERR_INVALID_DTYPE;
        if (N / 32 > UINT32_MAX / M) return Q_ERR_OVERFLOW;
        if (W->nb[0] != (size_t)(N / 32) * sizeof(q_block_q4_0)) return Q_ERR_INVALID_ARG;
        if (!W->data) return Q_ERR_INVALID_ARG;
        if (!aligned(W->data, 4)) return Q_ERR_MISALIGNED;
        segs[i] = GemvSeg{static_cast<const uint8_t*>(W->data), ys[i], residuals ? residuals[i] : nullptr, M};
    }
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(launch_gemv(segs, (int)n, Ws[0]->ne[1] / 32, static_cast<const uint4*>(workspace), (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_gemv_q4_f32_multi(const q_tensor* const* Ws, const float* const* residuals, float* const* ys,
                                  uint32_t n, const float* x, void* workspace, qh_stream s) {
    if (!Ws || !ys || !x) return Q_ERR_INVALID_ARG;
    if (n < 1 || n > 4) return Q_ERR_INVALID_SIZE;
    GemvSeg segs[4];
    for (uint32_t i = 0; i < n; ++i) {
        const q_tensor* W = Ws[i];
        if (!W) return Q_ERR_INVALID_ARG;
        QH_TRY_CODE(validate_gemv(W, x, ys[i]));
        if (W->ne[1] != Ws[0]->ne[1]) return Q_ERR_INVALID_SIZE;
        segs[i] = GemvSeg{static_cast<const uint8_t*>(W->data), ys[i], residuals ? residuals[i] : nullptr, W->ne[0]};
    }
    const uint32_t N = Ws[0]->ne[1];
    Device* d;
    QH_TRY_CODE(device(&d));
    if (!workspace && needs_workspace(N)) QH_TRY_CODE(library_workspace(d, N, &workspace));
    QH_TRY(launch_gemv_f32(segs, (int)n, N, x, static_cast<uint4*>(workspace), (hipStream_t)s));
    return Q_OK;
}

// Workspace of qh_gemv_q4_f32_softmax_argmax: the softmax's, then (at a
// 256-byte boundary) the GEMV's argmax partials.
static size_t lmhead_parts_offset(uint32_t M) { return (softmax_workspace_bytes(M) + 255) & ~(size_t)255; }

}  // extern "C"

namespace qh {

size_t gemv_softmax_ws_bytes(uint32_t M) {
    return lmhead_parts_offset(M) + (size_t)2 * kGemvAmaxMaxParts * sizeof(float);
}

q_error_code validate_gemv_softmax(const q_tensor* W, const float* x, const float* logits, const float* probs,
                                   const uint32_t* index_out, bool need_ws, const void* workspace) {
    QH_TRY_CODE(validate_gemv(W, x, logits));
    if (!probs || !index_out || (need_ws && !workspace)) return Q_ERR_INVALID_ARG;
    if (!aligned(probs, 32)) return Q_ERR_MISALIGNED;
    if (probs == logits || probs == x) return Q_ERR_ALIASING;
    return Q_OK;
}

q_error_code check_gemv_softmax_memory(const q_tensor* W, const float* x, const float* logits, const float* probs,
                                       const uint32_t* index_out, const void* workspace) {
    // Every operand must be device memory covering what the kernels touch:
    // a host or stale pointer becomes an error code, not a GPU fault.
    const uint32_t M = W->ne[0], N = W->ne[1];
    if (!device_range(W->data, (size_t)M * W->nb[0]) || !device_range(x, (size_t)N * 4) ||
        !device_range(logits, (size_t)M * 4) || !device_range(probs, (size_t)M * 4) ||
        !device_range(index_out, 4) || (workspace && !device_range(workspace, gemv_softmax_ws_bytes(M))))
        return fail(hipErrorInvalidValue,
                    "LM head: W->data, x, logits, probs, index_out or the workspace is not device memory of the "
                    "required size");
    return Q_OK;
}

q_error_code gemv_softmax_argmax_run(const q_tensor* W, const float* x, float* logits, float* probs,
                                     uint32_t* index_out, void* workspace, bool may_allocate, hipStream_t st) {
    const uint32_t M = W->ne[0], N = W->ne[1];
    float* ws = static_cast<float*>(workspace);
    float* parts = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + lmhead_parts_offset(M));
    const GemvSeg seg{static_cast<const uint8_t*>(W->data), logits, nullptr, M};
    uint32_t n_part = 0;
    hipError_t e = softmax_argmax_takes_parts(M)
                       ? launch_gemv_f32_amax(seg, N, x, nullptr, parts, kGemvAmaxMaxParts, &n_part, st)
                       : hipErrorNotSupported;
    if (e == hipSuccess) {
        QH_TRY(launch_softmax_argmax_parts(logits, probs, M, ws, parts, reinterpret_cast<const uint32_t*>(parts) + n_part,
                                           n_part, index_out, st));
        return Q_OK;
    }
    if (e != hipErrorNotSupported) QH_TRY(e);
    void* gws = nullptr;
    if (needs_workspace(N)) {
        if (!may_allocate) return fail(hipErrorInvalidValue, "input wider than the in-kernel digit conversion");
        Device* d;
        QH_TRY_CODE(device(&d));
        QH_TRY_CODE(library_workspace(d, N, &gws));
    }
    QH_TRY(launch_gemv_f32(&seg, 1, N, x, static_cast<uint4*>(gws), st));
    QH_TRY(launch_softmax_argmax_ws(logits, probs, M, ws, index_out, st));
    return Q_OK;
}

}  // namespace qh

extern "C" {

size_t qh_gemv_softmax_workspace_bytes(uint32_t M) { return gemv_softmax_ws_bytes(M); }

q_error_code qh_gemv_q4_f32_softmax_argmax(const q_tensor* W, const float* x, float* logits, float* probs,
                                           uint32_t* index_out, void* workspace, qh_stream s) {
    QH_TRY_CODE(validate_gemv_softmax(W, x, logits, probs, index_out, true, workspace));
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY_CODE(check_gemv_softmax_memory(W, x, logits, probs, index_out, workspace));
    return gemv_softmax_argmax_run(W, x, logits, probs, index_out, workspace, true, (hipStream_t)s);
}

size_t qh_gemm_workspace_bytes(uint32_t N, uint32_t T, uint32_t M_total) {
    return gemm_workspace_bytes(N, T, M_total);
}

q_error_code qh_gemm_q4_f32_multi(const q_tensor* const* Ws, float* const* Ys, uint32_t n, const float* X,
                                  uint32_t T, void* workspace, qh_stream s) {
    if (!Ws) return Q_ERR_INVALID_ARG;
    if (n < 1 || n > 3) return Q_ERR_INVALID_SIZE;
    const uint8_t* w[3];
    float* y[3];
    uint32_t M[3];
    uint32_t M_total = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const q_tensor* W = Ws[i];
        if (!W || !Ys || !Ys[i] || !X) return Q_ERR_INVALID_ARG;
        if (!aligned(X, 16) || !aligned(Ys[i], 4)) return Q_ERR_MISALIGNED;
        const uint32_t Mi = W->ne[0], N = W->ne[1];
        if (Mi == 0 || N == 0 || N % 32 != 0 || N > 32768 || N != Ws[0]->ne[1] || T == 0) return Q_ERR_INVALID_SIZE;
        if (W->type != Q_Q4_0) return Q_ERR_INVALID_DTYPE;
        if (N / 32 > UINT32_MAX / Mi || (uint64_t)Mi * (N / 32) * 20u >= (1ull << 31)) return Q_ERR_OVERFLOW;
        if (W->nb[0] != (size_t)(N / 32) * sizeof(q_block_q4_0)) return Q_ERR_INVALID_ARG;
        if (!W->data) return Q_ERR_INVALID_ARG;
        if (!aligned(W->data, 4)) return Q_ERR_MISALIGNED;
        // Y must not overlap X (the kernel reads X after writing Y tiles).
        const uintptr_t x0 = reinterpret_cast<uintptr_t>(X), x1 = x0 + (size_t)T * N * 4;
        const uintptr_t y0 = reinterpret_cast<uintptr_t>(Ys[i]), y1 = y0 + (size_t)T * Mi * 4;
        if (y0 < x1 && x0 < y1) return Q_ERR_ALIASING;
        w[i] = static_cast<const uint8_t*>(W->data);
        y[i] = Ys[i];
        M[i] = Mi;
        M_total += Mi;
    }
    if (!workspace) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    // Every operand must be device memory covering the whole extent the
    // kernels touch: a host or stale pointer becomes an error code here, not
    // a fault in the kernel.
    const uint32_t N = Ws[0]->ne[1];
    if (!device_range(X, (size_t)T * N * 4) ||
        !device_range(workspace, gemm_workspace_bytes(N, T, M_total)))
        return fail(hipErrorInvalidValue, "qh_gemm: X or workspace is not device memory of the required size");
    for (uint32_t i = 0; i < n; ++i) {
        if (!device_range(w[i], (size_t)M[i] * Ws[i]->nb[0]) || !device_range(y[i], (size_t)T * M[i] * 4))
            return fail(hipErrorInvalidValue, "qh_gemm: W->data or Y is not device memory of the required size");
    }
    QH_TRY(launch_gemm(w, y, M, (int)n, N, X, T, workspace, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_gemm_q4_f32(const q_tensor* W, const float* X, uint32_t T, float* Y, void* workspace,
                            qh_stream s) {
    if (!W) return Q_ERR_INVALID_ARG;
    return qh_gemm_q4_f32_multi(&W, &Y, 1, X, T, workspace, s);
}

// Reference src/ops/avx2/dequantize.c:82-96: silent return on NULL.
void q_dequantize_q4_0_block_avx2_public(const q_block_q4_0* __restrict__ block, float* __restrict__ output) {
    if (!block || !output) return;
    Device* d;
    if (device(&d) != Q_OK) return;
    std::lock_guard<std::mutex> lk(d->mu);
    void* buf;
    if (stage(d, 0, 256, &buf) != Q_OK) return;
    uint8_t* dblk = static_cast<uint8_t*>(buf);
    float* dout = reinterpret_cast<float*>(dblk + 64);
    if (hipMemcpyAsync(dblk, block, 20, hipMemcpyHostToDevice, d->stream) != hipSuccess) return;
    if (launch_dequant(dblk, dout, 1, d->stream) != hipSuccess) return;
    if (hipMemcpyAsync(output, dout, 128, hipMemcpyDeviceToHost, d->stream) != hipSuccess) return;
    (void)hipStreamSynchronize(d->stream);
}

// Reference src/ops/avx2/matmul.c:98-271 (host pointers, synchronous).
q_error_code q_gemv_q4_f32_avx2(const q_tensor* __restrict__ weights, const float* __restrict__ input,
                                float* __restrict__ output) {
    QH_TRY_CODE(validate_gemv(weights, input, output));
    Device* d;
    QH_TRY_CODE(device(&d));
    std::lock_guard<std::mutex> lk(d->mu);
    const uint32_t M = weights->ne[0], N = weights->ne[1];
    const size_t wbytes = (size_t)M * weights->nb[0];
    const void* wdev = resident_alias(weights->data, wbytes);
    hipStream_t s = d->stream;
    if (!wdev) {
        void* wbuf;
        QH_TRY_CODE(stage(d, 0, wbytes, &wbuf));
        QH_TRY(hipMemcpyAsync(wbuf, weights->data, wbytes, hipMemcpyHostToDevice, s));
        wdev = wbuf;
    }
    const size_t xb = ((size_t)N * 4 + 255) & ~(size_t)255;
    void* vbuf;
    QH_TRY_CODE(stage(d, 1, xb + (size_t)M * 4, &vbuf));
    float* dx = static_cast<float*>(vbuf);
    float* dy = reinterpret_cast<float*>(static_cast<uint8_t*>(vbuf) + xb);
    void* ws = nullptr;
    if (needs_workspace(N)) QH_TRY_CODE(stage(d, 2, qh_gemv_workspace_bytes(N), &ws));
    QH_TRY(hipMemcpyAsync(dx, input, (size_t)N * 4, hipMemcpyHostToDevice, s));
    QH_TRY_CODE(gemv_device(weights, wdev, dx, nullptr, dy, ws, s));
    QH_TRY(hipMemcpyAsync(output, dy, (size_t)M * 4, hipMemcpyDeviceToHost, s));
    QH_TRY(hipStreamSynchronize(s));
    return Q_OK;
}

}  // extern "C"
