// qh_kernels.hpp -- host-side launchers of the gfx950 kernels.  Launchers
// assume validated arguments (the C-ABI layer checks them) and return the
// hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qh {

// ---- Q4_0 ----

// Dequantize n_blocks 20-byte blocks into 32*n_blocks floats (bit-exact).
hipError_t launch_dequant(const uint8_t* blocks, float* out, uint64_t n_blocks, hipStream_t s);

// x-digit planes ("xd"): per 32-element block of x, the signed 4-bit digits
// of round(x * 2^k) in 6 planes (uint4 each), a meta word (k, NaN-injection
// word, wide flag, 0), and 6 planes of the residual's digits for blocks
// holding an outlier (qh_digits.hpp).  Layout: uint4 xd[13][nblk_pad];
// plane t of block c at xd[t * nblk_pad + c].
constexpr int kXdPlanes = 13;
inline uint32_t xd_pad(uint32_t nblk) { return (nblk + 63u) & ~63u; }
inline size_t xd_bytes(uint32_t nblk) { return (size_t)kXdPlanes * xd_pad(nblk) * 16u; }

// Fused RMSNorm (optional) + digit-plane preparation of an input vector.
// With norm_w != nullptr: h = rmsnorm(x, norm_w, eps) (reference order) is
// written to h_out (if non-null) and its digits to xd; else x's digits.
hipError_t launch_xprep(const float* x, uint32_t N, const float* norm_w, float eps, float* h_out,
                        uint4* xd, hipStream_t s);

// One GEMV "segment": rows [0, M) of a Q4_0 matrix with N = 32*nblk columns.
struct GemvSeg {
    const uint8_t* w;     // device AoS blocks
    float* y;             // output [M]
    const float* res;     // optional residual [M] (y = res + W.x)
    uint32_t M;
    // Decode-step epilogue (hd == 0: plain contiguous store).  With hd > 0
    // output row r is stored at y + pos*pos_stride + (r/hd)*head_stride +
    // r%hd, pos read from GemvDecode::pos; with rope the pair (r&~1, r|1) is
    // first rotated by the tables at row pos (reference src/ops/avx2/rope.c).
    uint32_t hd = 0;
    uint32_t head_stride = 0;
    uint32_t pos_stride = 0;
    bool rope = false;
};

// Device-side state read by decode-step epilogues.
struct GemvDecode {
    const uint32_t* pos = nullptr;  // current position (device)
    const float* cos_tab = nullptr; // [max_seq][hd] duplicated-pair tables
    const float* sin_tab = nullptr;
    // Optional RMSNorm factor: when in_part is set (per-block sums of squares
    // of the un-normalized input whose digits are given), every row value is
    // multiplied by newton(rsqrt(sum/N + eps)) before the epilogue.
    const float* in_part = nullptr;
    float eps = 0.0f;
    // fp32-input GEMV only: RMSNorm weight of x.  The kernel then converts
    // x*norm_w and scales every row by newton(rsqrt(sum(x^2)/N + eps)).
    const float* norm_w = nullptr;
};

// y = W . x for up to 4 segments sharing the same x (digit planes xd).
hipError_t launch_gemv(const GemvSeg* segs, int nseg, uint32_t nblk, const uint4* xd,
                       hipStream_t s, const GemvDecode* dec = nullptr);
// Same from the fp32 input x[N]: inputs of up to kGemvF32MaxBlk 32-element
// blocks are converted to digit planes inside the GEMV launch; wider ones
// are prepared into ws (xd_bytes(N/32) bytes) by a separate launch first.
constexpr uint32_t kGemvF32MaxBlk = 512;
// h[M] = silu(W_gate . n) * (W_up . n) with n = RMSNorm(x, norm_w, eps) made
// in the GEMV's prologue (x fp32, N <= 4096): the decode step's FFN input.
hipError_t launch_gemv_swiglu(const uint8_t* w_gate, const uint8_t* w_up, uint32_t M, uint32_t N, const float* x,
                              const float* norm_w, float eps, float* h, hipStream_t s);
hipError_t launch_gemv_f32(const GemvSeg* segs, int nseg, uint32_t N, const float* x, uint4* ws,
                           hipStream_t s, const GemvDecode* dec = nullptr);
// LM-head form (one segment, plain store, 2048 < N <= 4096, optional
// RMSNorm of x through dec->norm_w): also writes the greedy argmax's
// partials of y to amax (values [0, n), first indices [n, 2n) as uint32),
// n = *n_part <= cap, for launch_argmax_parts / launch_softmax_argmax_parts.
// hipErrorNotSupported for other shapes.
constexpr uint32_t kGemvAmaxMaxParts = 1024;
hipError_t launch_gemv_f32_amax(const GemvSeg& seg, uint32_t N, const float* x, const GemvDecode* dec, float* amax,
                                uint32_t cap, uint32_t* n_part, hipStream_t s);

// ---- batched prefill GEMM (k_gemm.hip) ----
// Y_i[t][m] = sum_k W_i[m][k] X[t][k] for nseg (1 to 3) matrices sharing
// X [T][N] (row-major fp32); Y_i is [T][M_i].  ws: gemm_workspace_bytes.
size_t gemm_workspace_bytes(uint32_t N, uint32_t T, uint32_t M_total);
hipError_t launch_gemm(const uint8_t* const* w, float* const* y, const uint32_t* M, int nseg, uint32_t N,
                       const float* X, uint32_t T, void* ws, hipStream_t s);
// The general form: up to 3 weight matrices, an optional residual per
// output (Y_i = R_i + W_i . x, R_i may equal Y_i), and the GEMM's rows x
// taken as X (plain), RMSNorm(X) * norm_w, or silu(X) * U (X the gate
// rows): the prefill layer's norms and SwiGLU product are made where the
// rows are converted for the matrix cores.
struct GemmSegs {
    int n = 0;
    const uint8_t* w[3] = {};
    float* y[3] = {};
    const float* res[3] = {};
    uint32_t M[3] = {};
};
// A GEMM with a K split can leave its reduction to the next kernel
// (launch_gemm_ex with defer_out; one matrix, or several without
// residuals): a one-matrix producer to the next GEMM's row conversion, where
// the partials, the per-token scale and the residual are summed in the
// reduction's own order (bit-identical), the rows written to y, and then
// converted; the prefill's Q|K|V to the RoPE / KV-cache pass.  valid is
// false when the launch had no split (y is then already written).
struct GemmDeferred {
    bool valid = false;
    const float* part = nullptr;   // [split][T][M]
    uint32_t split = 0, T = 0, M = 0;
    const float2* meta = nullptr;  // the producer's per-token (2^-e, non-finite flag)
    const float* res = nullptr;    // its residual rows [T][M] (or null)
    float* y = nullptr;            // its output rows [T][M] (one matrix; else null)
    const void* ws = nullptr;      // its workspace and staged row length
    uint32_t n_pad = 0;
};
struct GemmRows {
    const float* x = nullptr;       // [T][N]
    const float* u = nullptr;       // SwiGLU mode: [T][N] up rows
    const float* norm_w = nullptr;  // RMSNorm mode: [N] weight
    float eps = 0.0f;
    uint32_t T = 0, N = 0;
    // When set and valid, the rows are the deferred producer's y (x unused):
    // N must equal its M, and a shared workspace needs this GEMM's staged
    // rows no longer than the producer's (its partials lie beyond them).
    const GemmDeferred* from = nullptr;
};
hipError_t launch_gemm_ex(const GemmSegs& segs, const GemmRows& rows, void* ws, hipStream_t s,
                          GemmDeferred* defer_out = nullptr);

// ---- vector kernels (k_vec.hip) ----
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t N, float eps, hipStream_t s);
// RoPE of n_vec consecutive vectors of length N with one cos/sin table pair.
hipError_t launch_rope(const float* x, const float* ct, const float* st, float* y, uint32_t N,
                       uint32_t n_vec, hipStream_t s);
// Elements above the diagonal of an n x n matrix (row stride ld) := mask_value.
hipError_t launch_causal_mask(float* m, uint32_t n, uint32_t ld, float mask_value, hipStream_t s);
// y = silu(x) (u == nullptr) or silu(x) * u.
hipError_t launch_silu(const float* x, const float* u, float* y, uint32_t N, hipStream_t s);
hipError_t launch_softmax(const float* x, float* y, uint32_t N, hipStream_t s);
// Softmax in the reference's exact summation order (k_sample.hip): bit-exact
// with q_softmax_f32_avx2 except where the N % 8 tail's libm expf differs
// from the device's.  ws holds softmax_exact_ws_bytes(N) bytes (less, down
// to its dense minimum, makes the sum dense); x may alias y.
size_t softmax_exact_ws_bytes(uint32_t N);
hipError_t launch_softmax_exact(const float* x, float* y, uint32_t N, void* ws, size_t ws_bytes, hipStream_t s);
// op 0: o = a + b; op 1: o = a * b.
hipError_t launch_binary(const float* a, const float* b, float* o, uint32_t N, int op, hipStream_t s);
hipError_t launch_argmax(const float* x, uint32_t N, uint32_t* out, hipStream_t s);
// Multi-workgroup softmax / argmax for large N with a device workspace of
// softmax_workspace_bytes(N) / argmax_workspace_bytes(N) bytes (ws may be
// null, or N small: then the one-workgroup kernels run).  The argmax form
// also advances *pos_inout and appends to hist when those are non-null.
size_t softmax_workspace_bytes(uint32_t N);
size_t argmax_workspace_bytes(uint32_t N);
hipError_t launch_softmax_ws(const float* x, float* y, uint32_t N, float* ws, hipStream_t s);
// Softmax of x into y and the greedy argmax of x into *index_out (device),
// in the softmax's passes when N is large enough for its multi-workgroup
// form; ws as for launch_softmax_ws; x must not alias y.
hipError_t launch_softmax_argmax_ws(const float* x, float* y, uint32_t N, float* ws, uint32_t* index_out,
                                    hipStream_t s);
hipError_t launch_argmax_ws(const float* x, uint32_t N, uint32_t* out, uint32_t* pos_inout, uint32_t* hist,
                            uint32_t* hist_n, uint32_t hist_cap, float* ws, hipStream_t s);
// The same two results from Gm precomputed argmax partials (values parts[0,
// Gm), first indices [Gm, 2Gm) as uint32; launch_gemv_f32_amax): the argmax
// alone in one launch, or softmax + argmax in two (Gm <= 1024, N large
// enough for the multi-workgroup softmax; ws as for launch_softmax_ws).
hipError_t launch_argmax_parts(const float* x, uint32_t N, const float* parts, uint32_t Gm, uint32_t* out,
                               uint32_t* pos_inout, uint32_t* hist, uint32_t* hist_n, uint32_t hist_cap,
                               hipStream_t s);
bool softmax_argmax_takes_parts(uint32_t N);  // N large enough for launch_softmax_argmax_parts
hipError_t launch_softmax_argmax_parts(const float* x, float* y, uint32_t N, float* ws, const float* pmax,
                                       const uint32_t* pfirst, uint32_t Gm, uint32_t* index_out, hipStream_t s);
// C[M x N] (row stride ldc) = A (row stride lda) . B, B[k*ldb + j] or, with
// bt, B[j*K + k]; reference dot order.
hipError_t launch_matmul_f32(const float* A, uint32_t lda, const float* B, uint32_t ldb, bool bt, float* C,
                             uint32_t ldc, uint32_t M, uint32_t N, uint32_t K, hipStream_t s);

}  // namespace qh
