// qh_vec.hpp -- device helpers shared by the vector kernels: the reference's
// polynomial exp and the workgroup reductions.  Header-only, HIP device code.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qh {

// Polynomial exp of reference src/ops/avx2/avx_math.h:10-61, bit-exact:
// flags on the unclamped x (ordered compares), clamp with x86 minps/maxps
// semantics ((a<b)?a:b, (a>b)?a:b), degree-5 Horner in fmaf, max(r,0),
// x < -10 -> 0, x > 10 -> 22026.  (Host-callable too, for the exhaustive
// host check of the two forms below.)
__host__ __device__ __forceinline__ float exp_approx(float x) {
    const bool very_neg = x < -10.0f;
    const bool very_pos = x > 10.0f;
    float t = (x < 5.0f) ? x : 5.0f;
    t = (t > -5.0f) ? t : -5.0f;
    float r = 0.00833333f;
    r = fmaf(r, t, 0.04166667f);
    r = fmaf(r, t, 0.16666667f);
    r = fmaf(r, t, 0.5f);
    r = fmaf(r, t, 1.0f);
    r = fmaf(r, t, 1.0f);
    r = (r > 0.0f) ? r : 0.0f;
    if (very_neg) r = 0.0f;
    if (very_pos) r = 22026.0f;
    return r;
}

// exp_approx for x <= 0 or NaN (a softmax argument s - max s), the same
// values without the +-10 flags: x <= -10 already gives 0 (t clamps to -5,
// where the polynomial is -12.33, and max(r, 0) is 0) and x > 10 cannot
// occur; a NaN takes t = 5 in both (91.41).
__host__ __device__ __forceinline__ float exp_approx_nonpos(float x) {
    float t = (x < 5.0f) ? x : 5.0f;
    t = (t > -5.0f) ? t : -5.0f;
    float r = 0.00833333f;
    r = fmaf(r, t, 0.04166667f);
    r = fmaf(r, t, 0.16666667f);
    r = fmaf(r, t, 0.5f);
    r = fmaf(r, t, 1.0f);
    r = fmaf(r, t, 1.0f);
    return (r > 0.0f) ? r : 0.0f;
}

// SiLU of reference src/ops/avx2/silu.c:75-82 (vector part).
__device__ __forceinline__ float silu_approx(float x) {
    const float e = exp_approx(-x);
    const float d = 1.0f + e;
    const float sg = 1.0f / d;
    return x * sg;
}

// Fixed-order workgroup sum for blockDim.x == NT (multiple of 64): wave
// butterflies, then the wave partials in index order.  Every thread gets the
// result.  `red` needs NT/64 floats of shared memory.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) s += red[i];
    __syncthreads();
    return s;
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) s = fmaxf(s, red[i]);
    __syncthreads();
    return s;
}

// RMSNorm scale r for x[0..N), N % 4 == 0 (fixed-order tree sum of squares:
// each thread accumulates its float4s (4 lane partials), then the lanes of
// the float4, then block_sum; mean = sum/(float)N; a = mean + eps;
// r0 = rsq(a); one Newton step (r0*(3 - a*(r0*r0)))*0.5 as in reference
// src/ops/avx2/rmsnorm.c:62-71).  Loads are issued 4 at a time so a thread
// keeps several in flight.
template <int NT>
__device__ __forceinline__ float rms_scale(const float* __restrict__ x, uint32_t N, float eps, float* red) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const uint32_t n4 = N / 4;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    uint32_t i = threadIdx.x;
    for (; i + 3 * NT < n4; i += 4 * NT) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = x4[i + u * NT];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            s0 = s0 + v[u].x * v[u].x;
            s1 = s1 + v[u].y * v[u].y;
            s2 = s2 + v[u].z * v[u].z;
            s3 = s3 + v[u].w * v[u].w;
        }
    }
    for (; i < n4; i += NT) {
        const float4 v = x4[i];
        s0 = s0 + v.x * v.x;
        s1 = s1 + v.y * v.y;
        s2 = s2 + v.z * v.z;
        s3 = s3 + v.w * v.w;
    }
    const float ss = (s0 + s1) + (s2 + s3);
    const float sum = block_sum<NT>(ss, red);
    const float mean = sum / (float)N;
    const float a = mean + eps;
    const float r0 = __builtin_amdgcn_rsqf(a);
    const float rr = r0 * r0;
    const float ar = a * rr;
    const float t = 3.0f - ar;
    const float r1 = r0 * t;
    return r1 * 0.5f;
}

// Total order of the greedy argmax's candidates (value, index) on non-NaN
// values: the larger value, on equal values the smaller index; a NaN never
// wins.  Combining per-subset winners with it gives the first index of the
// maximum whatever the subsets and their order.
__device__ __forceinline__ bool arg_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

}  // namespace qh
