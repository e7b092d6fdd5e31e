// k_vec.hip -- vector kernels of the decode step for gfx950: RMSNorm, RoPE,
// SiLU (and the fused SwiGLU product), softmax, add, mul, argmax.
//
// Bit-exactness with the reference: RoPE, add, mul, the polynomial exp, the
// vector part of SiLU and every per-element softmax step are the same IEEE
// operations in the same order, so they are bit-exact.  Reductions (the
// RMSNorm sum of squares, the softmax sum) use a fixed tree instead of the
// reference's 8 sequential lane chains, so their last bit can differ; the
// reference's RMSNorm bits are CPU-specific anyway (rsqrtps seed).  The
// N%8 tails of SiLU/softmax call the device expf where the reference calls
// glibc expf (parity at that libm boundary is tolerance-only).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "qh_kernels.hpp"
#include "qh_vec.hpp"

namespace qh {

constexpr uint32_t kSmxSlice = 2048;       // elements per workgroup slice (multi-workgroup path)
constexpr uint32_t kSmxMaxSlices = 1024;   // slices are widened beyond this many
constexpr uint32_t kSmxMultiMin = 16384;   // below this N one workgroup is faster
constexpr int kVecThreads = 1024;

// RMSNorm, one workgroup of 256 threads: y = (x*r)*w (reference
// src/ops/avx2/rmsnorm.c:166-176).  Same reduction as the fused
// RMSNorm + digit-prep kernel, so both give identical bits.
constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(const float* __restrict__ x,
                                                          const float* __restrict__ w, float* __restrict__ y,
                                                          uint32_t N, float eps) {
    __shared__ float red[kNormThreads / 64];
    const float r = rms_scale<kNormThreads>(x, N, eps, red);
    for (uint32_t i = threadIdx.x; i < N; i += kNormThreads) {
        const float n = x[i] * r;
        y[i] = n * w[i];
    }
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t N, float eps, hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), 0, s, x, w, y, N, eps);
    return hipGetLastError();
}

// RoPE over n_vec vectors of length N sharing one table pair
// (reference src/ops/avx2/rope.c:244-285): y0 = x0*c - x1*s, y1 = x1*c + x0*s.
__global__ __launch_bounds__(256) void k_rope(const float* __restrict__ x, const float* __restrict__ ct,
                                              const float* __restrict__ st, float* __restrict__ y,
                                              uint32_t N, uint32_t total_pairs) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= total_pairs) return;
    const uint32_t half = N / 2;
    const uint32_t v = p / half, i = 2 * (p % half);
    const float2 xv = *reinterpret_cast<const float2*>(x + (size_t)v * N + i);
    const float c = ct[i], sn = st[i];
    const float a0 = xv.x * c, b0 = xv.y * sn;
    const float a1 = xv.y * c, b1 = xv.x * sn;
    *reinterpret_cast<float2*>(y + (size_t)v * N + i) = make_float2(a0 - b0, a1 + b1);
}

hipError_t launch_rope(const float* x, const float* ct, const float* st, float* y, uint32_t N, uint32_t n_vec,
                       hipStream_t s) {
    const uint32_t total = (N / 2) * n_vec;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope, dim3((total + 255) / 256), dim3(256), 0, s, x, ct, st, y, N, total);
    return hipGetLastError();
}

// Causal mask (reference src/ops/avx2/causal_mask_fp32.c:16-138): every
// element above the diagonal of the n x n matrix (row stride ld floats) is
// set to mask_value; the diagonal, the lower triangle and the columns past n
// keep their bits.  One workgroup per row, float stores only.
__global__ __launch_bounds__(256) void k_causal_mask(float* __restrict__ m, uint32_t n, uint32_t ld, float v) {
    const uint32_t i = blockIdx.x;
    float* row = m + (size_t)i * ld;
    for (uint32_t j = i + 1u + threadIdx.x; j < n; j += 256) row[j] = v;
}

hipError_t launch_causal_mask(float* m, uint32_t n, uint32_t ld, float mask_value, hipStream_t s) {
    if (n < 2) return hipSuccess;
    hipLaunchKernelGGL(k_causal_mask, dim3(n - 1), dim3(256), 0, s, m, n, ld, mask_value);
    return hipGetLastError();
}

// SiLU (reference src/ops/avx2/silu.c:44-91).  With u != nullptr the output
// is silu(x)*u, the SwiGLU product of reference src/models/model.c:1516-1549.
__global__ __launch_bounds__(256) void k_silu(const float* __restrict__ x, const float* __restrict__ u,
                                              float* __restrict__ y, uint32_t N) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const uint32_t nv = (N >= 8) ? (N & ~7u) : 0u;
    const float xv = x[i];
    float r;
    if (i < nv) {
        r = silu_approx(xv);
    } else {
        const float sg = 1.0f / (1.0f + expf(-xv));
        r = xv * sg;
    }
    y[i] = u ? r * u[i] : r;
}

hipError_t launch_silu(const float* x, const float* u, float* y, uint32_t N, hipStream_t s) {
    if (N == 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu, dim3((N + 255) / 256), dim3(256), 0, s, x, u, y, N);
    return hipGetLastError();
}

// Softmax, one workgroup (reference src/ops/avx2/softmax.c:30-213).
// N >= 8: m = max; e_i = exp_approx(x_i - m) for i < N&~7 (tree sum), tail
// e_i = expf(x_i - m) added in index order after the vector sum, inv =
// 1/sum, y_i = e_i*inv.  N < 8: expf, sequential sum, y_i = e_i/sum.
// x may alias y.
__global__ __launch_bounds__(kVecThreads) void k_softmax(const float* x, float* y, uint32_t N) {
    __shared__ float red[kVecThreads / 64];
    if (N < 8) {
        if (threadIdx.x == 0) {
            float mx = x[0];
            for (uint32_t i = 1; i < N; ++i)
                if (x[i] > mx) mx = x[i];
            float e[8];
            float sum = 0.0f;
            for (uint32_t i = 0; i < N; ++i) {
                e[i] = expf(x[i] - mx);
                sum += e[i];
            }
            for (uint32_t i = 0; i < N; ++i) y[i] = e[i] / sum;
        }
        return;
    }
    const uint32_t nv = N & ~7u;
    float m = -INFINITY;
    for (uint32_t i = threadIdx.x; i < N; i += kVecThreads) m = fmaxf(m, x[i]);
    m = block_max<kVecThreads>(m, red);
    float ls = 0.0f;
    for (uint32_t i = threadIdx.x; i < nv; i += kVecThreads) {
        const float d = x[i] - m;
        const float e = exp_approx(d);
        ls = ls + e;
        y[i] = e;
    }
    if (threadIdx.x == 0) {
        for (uint32_t i = nv; i < N; ++i) y[i] = expf(x[i] - m);
    }
    float sum = block_sum<kVecThreads>(ls, red);  // its barriers publish the tail values
    // Sequential tail additions after the vector sum, in index order.
    for (uint32_t i = nv; i < N; ++i) sum = sum + y[i];
    __syncthreads();  // every thread has read the tails before any is rescaled
    const float inv = 1.0f / sum;
    for (uint32_t i = threadIdx.x; i < N; i += kVecThreads) y[i] = y[i] * inv;
}

hipError_t launch_softmax(const float* x, float* y, uint32_t N, hipStream_t s) {
    if (N == 0) return hipSuccess;
    hipLaunchKernelGGL(k_softmax, dim3(1), dim3(kVecThreads), 0, s, x, y, N);
    return hipGetLastError();
}

// Multi-workgroup softmax for large N (same semantics as k_softmax, N >= 8):
//   A: per-slice max over all N elements;
//   B: global max (exact, any order), e_i = exp_approx(x_i - m) for i <
//      N&~7 written to y with a per-slice fixed-order sum; tail e_i =
//      expf(x_i - m) written to y and kept in the workspace;
//   C: total = per-slice sums in slice order, then the tail values in index
//      order; inv = 1/total; y_i *= inv.
// Workspace floats: [0, G) slice max, [G, 2G) slice sums, [2G, 2G+8) tail,
// [2G+8, 3G+8) the slices' first max indices (fused argmax).
// With first_idx: also the first index of the slice holding its maximum
// (0xFFFFFFFF when no element equals it, e.g. an all-NaN slice).
// A thread's elements of a slice are base, base + 256, ... < b1; they are
// loaded kSmxUnroll at a time, all loads issued before any value is used
// (one memory round trip per chunk instead of one per element).
constexpr int kSmxUnroll = kSmxSlice / 256;

__device__ __forceinline__ void load_slice_chunk(const float* x, uint32_t base, uint32_t b1,
                                                 float (&v)[kSmxUnroll]) {
#pragma unroll
    for (int u = 0; u < kSmxUnroll; ++u) {
        const uint32_t i = base + 256u * u;
        v[u] = i < b1 ? x[i] : 0.0f;
    }
}

__global__ __launch_bounds__(256) void k_smx_max(const float* x, uint32_t N, uint32_t slice, float* ws,
                                                 uint32_t* first_idx) {
    __shared__ float red[4];
    __shared__ uint32_t redi[4];
    const uint32_t b0 = blockIdx.x * slice, b1 = min(N, b0 + slice);
    if (!first_idx) {
        float m = -INFINITY;
        for (uint32_t base = b0 + threadIdx.x; base < b1; base += 256u * kSmxUnroll) {
            float v[kSmxUnroll];
            load_slice_chunk(x, base, b1, v);
#pragma unroll
            for (int u = 0; u < kSmxUnroll; ++u)
                if (base + 256u * u < b1) m = fmaxf(m, v[u]);
        }
        m = block_max<256>(m, red);
        if (threadIdx.x == 0) ws[blockIdx.x] = m;
        return;
    }
    // One pass: each thread's (max, first index holding it) over its
    // elements in increasing index order (NaN never compares greater), then
    // the larger value or, on equal values, the smaller index.  The value
    // is the same max as the fmaxf form above.
    float m = -INFINITY;
    uint32_t f = 0xFFFFFFFFu;
    for (uint32_t base = b0 + threadIdx.x; base < b1; base += 256u * kSmxUnroll) {
        float v[kSmxUnroll];
        load_slice_chunk(x, base, b1, v);
#pragma unroll
        for (int u = 0; u < kSmxUnroll; ++u) {
            const uint32_t i = base + 256u * u;
            if (i < b1 && (v[u] > m || (f == 0xFFFFFFFFu && v[u] == m))) {
                m = v[u];
                f = i;
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float om = __shfl_xor(m, off);
        const uint32_t of = (uint32_t)__shfl_xor((int)f, off);
        if (om > m || (om == m && of < f)) {
            m = om;
            f = of;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = m;
        redi[threadIdx.x >> 6] = f;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        m = red[0];
        f = redi[0];
        for (int w = 1; w < 4; ++w)
            if (red[w] > m || (red[w] == m && redi[w] < f)) {
                m = red[w];
                f = redi[w];
            }
        ws[blockIdx.x] = m;
        first_idx[blockIdx.x] = f;
    }
}

// With index_out: workgroup 0 also writes the greedy argmax of x (reference
// src/main.c:870-881: first index of the maximum, strict >, index 0 when
// x[0] is NaN or nothing compares greater) from the slice maxima and their
// first indices, loaded with the maxima (slices are in index order: the
// smallest first index among the slices holding the global max is the first
// index overall).
// The maxima come as Gm partials pmax[0..Gm) (with first indices pfirst for
// the argmax): the slices' own from k_smx_max, or a producer's.
__global__ __launch_bounds__(256) void k_smx_exp(const float* x, float* y, uint32_t N, uint32_t slice, uint32_t G,
                                                 float* ws, const float* pmax, const uint32_t* first_idx,
                                                 uint32_t Gm, uint32_t* index_out) {
    __shared__ float red[4];
    __shared__ uint32_t redi[4];
    constexpr int kPerThread = (kSmxMaxSlices + 255) / 256;
    const bool arg = index_out && blockIdx.x == 0;
    const uint32_t b0 = blockIdx.x * slice, b1 = min(N, b0 + slice);
    // The slice's first chunk does not depend on the max: load it first.
    uint32_t base = b0 + threadIdx.x;
    float xv[kSmxUnroll];
    load_slice_chunk(x, base, b1, xv);
    float wv[kPerThread];
    uint32_t fv[kPerThread];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const uint32_t g = threadIdx.x + 256u * k;
        wv[k] = g < Gm ? pmax[g] : -INFINITY;
        fv[k] = (arg && g < Gm) ? first_idx[g] : 0xFFFFFFFFu;
        m = fmaxf(m, wv[k]);
    }
    m = block_max<256>(m, red);
    if (arg) {
        uint32_t best = 0xFFFFFFFFu;
#pragma unroll
        for (int k = 0; k < kPerThread; ++k)
            if (wv[k] == m && fv[k] < best) best = fv[k];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) best = min(best, (uint32_t)__shfl_xor((int)best, off));
        if ((threadIdx.x & 63) == 0) redi[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            best = min(min(redi[0], redi[1]), min(redi[2], redi[3]));
            if (best == 0xFFFFFFFFu || x[0] != x[0]) best = 0;
            *index_out = best;
        }
    }
    const uint32_t nv = N & ~7u;
    float ls = 0.0f;
    while (base < b1) {
#pragma unroll
        for (int u = 0; u < kSmxUnroll; ++u) {
            const uint32_t i = base + 256u * u;
            if (i < b1) {
                const float d = xv[u] - m;
                if (i < nv) {
                    const float e = exp_approx(d);
                    ls = ls + e;
                    y[i] = e;
                } else {
                    const float e = expf(d);
                    y[i] = e;
                    ws[2 * G + (i - nv)] = e;
                }
            }
        }
        base += 256u * kSmxUnroll;
        if (base < b1) load_slice_chunk(x, base, b1, xv);
    }
    const float sum = block_sum<256>(ls, red);
    if (threadIdx.x == 0) ws[G + blockIdx.x] = sum;
}

__global__ __launch_bounds__(256) void k_smx_norm(float* y, uint32_t N, uint32_t slice, uint32_t G,
                                                  const float* ws) {
    __shared__ float inv_s;
    const uint32_t b0 = blockIdx.x * slice, b1 = min(N, b0 + slice);
    uint32_t base = b0 + threadIdx.x;
    float yv[kSmxUnroll];
    load_slice_chunk(y, base, b1, yv);
    // total = slice sums in slice order, then the tail values in index order
    // (sequential adds).  Wave 0 loads them in parallel, lane l holding
    // entries l, l + 64, ...; the adds read them back lane by lane.
    if (threadIdx.x < 64) {
        constexpr int kPer = kSmxMaxSlices / 64;
        const uint32_t ln = threadIdx.x, nt = N - (N & ~7u);
        float pv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t g = (uint32_t)k * 64u + ln;
            pv[k] = g < G ? ws[G + g] : 0.0f;
        }
        const float tv = ln < nt ? ws[2 * G + ln] : 0.0f;
        float total = 0.0f;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t g0 = (uint32_t)k * 64u;
            if (g0 < G) {
                const uint32_t n = min(64u, G - g0);
                for (uint32_t l = 0; l < n; ++l)
                    total = total + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv[k]), (int)l));
            }
        }
        for (uint32_t l = 0; l < nt; ++l) total = total + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tv), (int)l));
        if (ln == 0) inv_s = 1.0f / total;
    }
    __syncthreads();
    const float inv = inv_s;
    while (base < b1) {
#pragma unroll
        for (int u = 0; u < kSmxUnroll; ++u) {
            const uint32_t i = base + 256u * u;
            if (i < b1) y[i] = yv[u] * inv;
        }
        base += 256u * kSmxUnroll;
        if (base < b1) load_slice_chunk(y, base, b1, yv);
    }
}

static void smx_shape(uint32_t N, uint32_t* slice, uint32_t* G) {
    uint32_t sl = kSmxSlice;
    while ((N + sl - 1) / sl > kSmxMaxSlices) sl *= 2;
    *slice = sl;
    *G = (N + sl - 1) / sl;
}

size_t softmax_workspace_bytes(uint32_t N) {
    uint32_t sl, G;
    smx_shape(N, &sl, &G);
    return ((size_t)4 * G + 8) * sizeof(float);
}

hipError_t launch_softmax_ws(const float* x, float* y, uint32_t N, float* ws, hipStream_t s) {
    if (N == 0) return hipSuccess;
    if (N < kSmxMultiMin || !ws) return launch_softmax(x, y, N, s);
    uint32_t sl, G;
    smx_shape(N, &sl, &G);
    hipLaunchKernelGGL(k_smx_max, dim3(G), dim3(256), 0, s, x, N, sl, ws, (uint32_t*)nullptr);
    hipLaunchKernelGGL(k_smx_exp, dim3(G), dim3(256), 0, s, x, y, N, sl, G, ws, (const float*)ws,
                       (const uint32_t*)nullptr, G, (uint32_t*)nullptr);
    hipLaunchKernelGGL(k_smx_norm, dim3(G), dim3(256), 0, s, y, N, sl, G, ws);
    return hipGetLastError();
}

// Softmax and greedy argmax of the same x in the softmax's three passes
// (the slice maxima carry their first indices).  x must not alias y.
hipError_t launch_softmax_argmax_ws(const float* x, float* y, uint32_t N, float* ws, uint32_t* index_out,
                                    hipStream_t s) {
    if (N == 0) return hipSuccess;
    if (N < kSmxMultiMin || !ws) {
        hipError_t e = launch_argmax(x, N, index_out, s);
        if (e != hipSuccess) return e;
        return launch_softmax(x, y, N, s);
    }
    uint32_t sl, G;
    smx_shape(N, &sl, &G);
    uint32_t* first = reinterpret_cast<uint32_t*>(ws + 2 * G + 8);
    hipLaunchKernelGGL(k_smx_max, dim3(G), dim3(256), 0, s, x, N, sl, ws, first);
    hipLaunchKernelGGL(k_smx_exp, dim3(G), dim3(256), 0, s, x, y, N, sl, G, ws, (const float*)ws,
                       (const uint32_t*)first, G, index_out);
    hipLaunchKernelGGL(k_smx_norm, dim3(G), dim3(256), 0, s, y, N, sl, G, ws);
    return hipGetLastError();
}

bool softmax_argmax_takes_parts(uint32_t N) { return N >= kSmxMultiMin; }

hipError_t launch_softmax_argmax_parts(const float* x, float* y, uint32_t N, float* ws, const float* pmax,
                                       const uint32_t* pfirst, uint32_t Gm, uint32_t* index_out, hipStream_t s) {
    if (N < kSmxMultiMin || !ws || !pmax || !pfirst || !index_out || Gm == 0 || Gm > kSmxMaxSlices)
        return hipErrorInvalidValue;
    uint32_t sl, G;
    smx_shape(N, &sl, &G);
    hipLaunchKernelGGL(k_smx_exp, dim3(G), dim3(256), 0, s, x, y, N, sl, G, ws, pmax, pfirst, Gm, index_out);
    hipLaunchKernelGGL(k_smx_norm, dim3(G), dim3(256), 0, s, y, N, sl, G, ws);
    return hipGetLastError();
}

// Elementwise add / mul (reference add_fp32.c:127-161, mul_fp32.c:89-123).
__global__ __launch_bounds__(256) void k_binary(const float* a, const float* b, float* o, uint32_t N, int op) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const float av = a[i], bv = b[i];
    o[i] = op == 0 ? av + bv : av * bv;
}

hipError_t launch_binary(const float* a, const float* b, float* o, uint32_t N, int op, hipStream_t s) {
    if (N == 0) return hipSuccess;
    hipLaunchKernelGGL(k_binary, dim3((N + 255) / 256), dim3(256), 0, s, a, b, o, N, op);
    return hipGetLastError();
}

// Greedy argmax (reference src/main.c:870-881): first index of the maximum
// under strict '>' scanning from index 0; NaN entries never win; a NaN at
// index 0 makes the answer 0 (arg_better, qh_vec.hpp).

// With pos_inout / hist (the on-device generation loop): also advance the
// position and append the token to hist[0..hist_cap).
__global__ __launch_bounds__(kVecThreads) void k_argmax(const float* __restrict__ x, uint32_t N,
                                                        uint32_t* __restrict__ out, uint32_t* __restrict__ pos_inout,
                                                        uint32_t* __restrict__ hist, uint32_t* __restrict__ hist_n,
                                                        uint32_t hist_cap) {
    __shared__ float sv[kVecThreads / 64];
    __shared__ uint32_t si[kVecThreads / 64];
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    // 8 loads in flight per thread per round.
    uint32_t i = threadIdx.x;
    for (; i + 7 * kVecThreads < N; i += 8 * kVecThreads) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = x[i + u * kVecThreads];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (arg_better(v[u], i + u * kVecThreads, bv, bi)) {
                bv = v[u];
                bi = i + u * kVecThreads;
            }
    }
    for (; i < N; i += kVecThreads) {
        const float v = x[i];
        if (arg_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = sv[0];
        uint32_t i = si[0];
        for (int k = 1; k < kVecThreads / 64; ++k)
            if (arg_better(sv[k], si[k], v, i)) {
                v = sv[k];
                i = si[k];
            }
        if (N > 0 && x[0] != x[0]) i = 0;  // NaN at index 0: nothing compares greater
        if (i == 0xFFFFFFFFu) i = 0;
        *out = i;
        if (pos_inout) *pos_inout += 1u;
        if (hist) {
            const uint32_t n = *hist_n;
            if (n < hist_cap) hist[n] = i;
            *hist_n = n + 1u;
        }
    }
}

hipError_t launch_argmax(const float* x, uint32_t N, uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(kVecThreads), 0, s, x, N, out, nullptr, nullptr, nullptr, 0u);
    return hipGetLastError();
}

hipError_t launch_argmax_step(const float* x, uint32_t N, uint32_t* tok_out, uint32_t* pos_inout, uint32_t* hist,
                              uint32_t* hist_n, uint32_t hist_cap, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(kVecThreads), 0, s, x, N, tok_out, pos_inout, hist, hist_n, hist_cap);
    return hipGetLastError();
}

// Multi-workgroup argmax: per-slice (value, first index) partials, then one
// workgroup combines them.  arg_better is a total order on non-NaN values
// (larger value, then smaller index), so the result does not depend on the
// combination order; NaN never wins, and a NaN at index 0 gives index 0 (no
// element compares greater than it, reference main.c:870-881).
// Workspace: floats [0, G) values, then uint32 [G, 2G) indices.
__global__ __launch_bounds__(256) void k_amax_part(const float* __restrict__ x, uint32_t N, uint32_t slice,
                                                   float* __restrict__ ws) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const uint32_t b0 = blockIdx.x * slice, b1 = min(N, b0 + slice);
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t base = b0 + threadIdx.x; base < b1; base += 256u * kSmxUnroll) {
        float v[kSmxUnroll];
        load_slice_chunk(x, base, b1, v);
#pragma unroll
        for (int u = 0; u < kSmxUnroll; ++u) {
            const uint32_t i = base + 256u * u;
            if (i < b1 && arg_better(v[u], i, bv, bi)) {
                bv = v[u];
                bi = i;
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = sv[0];
        uint32_t i = si[0];
        for (int k = 1; k < 4; ++k)
            if (arg_better(sv[k], si[k], v, i)) {
                v = sv[k];
                i = si[k];
            }
        ws[blockIdx.x] = v;
        reinterpret_cast<uint32_t*>(ws)[gridDim.x + blockIdx.x] = i;
    }
}

__global__ __launch_bounds__(256) void k_amax_final(const float* __restrict__ x, uint32_t N, uint32_t G,
                                                    const float* __restrict__ ws, uint32_t* __restrict__ out,
                                                    uint32_t* __restrict__ pos_inout, uint32_t* __restrict__ hist,
                                                    uint32_t* __restrict__ hist_n, uint32_t hist_cap) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const uint32_t* wi = reinterpret_cast<const uint32_t*>(ws) + G;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t g = threadIdx.x; g < G; g += 256) {
        const float v = ws[g];
        const uint32_t i = wi[g];
        if (arg_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = sv[0];
        uint32_t i = si[0];
        for (int k = 1; k < 4; ++k)
            if (arg_better(sv[k], si[k], v, i)) {
                v = sv[k];
                i = si[k];
            }
        if (x[0] != x[0]) i = 0;  // NaN at index 0: nothing compares greater
        if (i == 0xFFFFFFFFu) i = 0;
        *out = i;
        if (pos_inout) *pos_inout += 1u;
        if (hist) {
            const uint32_t n = *hist_n;
            if (n < hist_cap) hist[n] = i;
            *hist_n = n + 1u;
        }
    }
}

size_t argmax_workspace_bytes(uint32_t N) {
    uint32_t sl, G;
    smx_shape(N, &sl, &G);
    return (size_t)2 * G * sizeof(float);
}

hipError_t launch_argmax_ws(const float* x, uint32_t N, uint32_t* out, uint32_t* pos_inout, uint32_t* hist,
                            uint32_t* hist_n, uint32_t hist_cap, float* ws, hipStream_t s) {
    if (N < kSmxMultiMin || !ws) {
        hipLaunchKernelGGL(k_argmax, dim3(1), dim3(kVecThreads), 0, s, x, N, out, pos_inout, hist, hist_n, hist_cap);
        return hipGetLastError();
    }
    uint32_t sl, G;
    smx_shape(N, &sl, &G);
    hipLaunchKernelGGL(k_amax_part, dim3(G), dim3(256), 0, s, x, N, sl, ws);
    hipLaunchKernelGGL(k_amax_final, dim3(1), dim3(256), 0, s, x, N, G, ws, out, pos_inout, hist, hist_n, hist_cap);
    return hipGetLastError();
}

hipError_t launch_argmax_parts(const float* x, uint32_t N, const float* parts, uint32_t Gm, uint32_t* out,
                               uint32_t* pos_inout, uint32_t* hist, uint32_t* hist_n, uint32_t hist_cap,
                               hipStream_t s) {
    if (!x || N == 0 || !parts || Gm == 0 || !out) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_amax_final, dim3(1), dim3(256), 0, s, x, N, Gm, parts, out, pos_inout, hist, hist_n,
                       hist_cap);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fp32 matmul C = A . B in the reference dot order (matmul_fp32.c:302-468):
// per 32-element chunk of K, element k goes to accumulator c = (k%32)/8,
// lane l = k%8, with FMA; per lane S_l = (a0+a1)+(a2+a3); then
// ((S0+S4)+(S1+S5))+((S2+S6)+(S3+S7)) (hsum256_ps); then the K%32 tail
// sequentially as dot = dot + a*b (separately rounded).  Eight lanes per
// output element: lane l holds a[0..3][l]; the tree runs on DPP.
// B element (k, j) is B[k*ldb + j], or B[j*K + k] when bt (a transposed
// view, read with column stride K as the reference does).
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp_sel(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__global__ __launch_bounds__(256) void k_matmul_f32(const float* __restrict__ A, uint32_t lda,
                                                    const float* __restrict__ B, uint32_t ldb, uint32_t bt,
                                                    float* __restrict__ C, uint32_t ldc, uint32_t M, uint32_t N,
                                                    uint32_t K) {
    const uint64_t gid = ((uint64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const uint32_t l = threadIdx.x & 7;
    const bool valid = gid < (uint64_t)M * N;
    // Every lane of a group takes part in the DPP tree; a group past the end
    // computes element (0, 0) and does not store.
    const uint32_t i = valid ? (uint32_t)(gid / N) : 0u;
    const uint32_t j = valid ? (uint32_t)(gid % N) : 0u;
    const float* a = A + (size_t)i * lda;
    const float* bcol = bt ? B + (size_t)j * K : B + j;
    const size_t bstep = bt ? 1 : ldb;
    const uint32_t kv = K & ~31u;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t k = 0; k < kv; k += 32) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t kk = k + 8u * c + l;
            acc[c] = fmaf(a[kk], bcol[(size_t)kk * bstep], acc[c]);
        }
    }
    const float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    const float t = s + dpp_sel<0x104>(s);  // row_shl:4: l < 4 -> S_l + S_{l+4}
    const float u = t + dpp_sel<0xB1>(t);   // quad_perm [1,0,3,2]
    const float d = u + dpp_sel<0x4E>(u);   // quad_perm [2,3,0,1]: lane 0 holds the tree
    if (valid && l == 0) {
        float dot = kv > 0 ? d : 0.0f;
        for (uint32_t k = kv; k < K; ++k) {
            const float p = a[k] * bcol[(size_t)k * bstep];
            dot = dot + p;
        }
        C[(size_t)i * ldc + j] = dot;
    }
}

hipError_t launch_matmul_f32(const float* A, uint32_t lda, const float* B, uint32_t ldb, bool bt, float* C,
                             uint32_t ldc, uint32_t M, uint32_t N, uint32_t K, hipStream_t s) {
    const uint64_t threads = (uint64_t)M * N * 8;
    const uint64_t grid = (threads + 255) / 256;
    if (grid == 0) return hipSuccess;
    if (grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_matmul_f32, dim3((uint32_t)grid), dim3(256), 0, s, A, lda, B, ldb, bt ? 1u : 0u, C, ldc,
                       M, N, K);
    return hipGetLastError();
}

}  // namespace qh
