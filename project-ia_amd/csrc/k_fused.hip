// k_fused.hip -- the decode step's Wo and W_gate|W_up GEMVs with their
// neighbours folded into prologue and epilogue (no separate RMSNorm/digit
// or SwiGLU/digit kernels).
//
// Every workgroup owns one 32-row block of the output vector (64 matrix rows
// for W_gate|W_up: the same 32 rows of both), so the epilogue sees a whole
// 32-element block and can emit the next GEMV's digit planes itself:
//  * RESID  (Wo): x_new = res + W.x; stores x_new, the digit planes of
//    x_new * w_norm (the FFN RMSNorm's weight) and the block's sum of
//    squares of x_new.
//  * SWIGLU consumes such an input: the RMSNorm scale r = newton(rsqrt(sum/N
//    + eps)) (reference src/ops/avx2/rmsnorm.c:62-71) comes from the
//    producer's per-block sums (fixed order), and the matrix products are
//    scaled by r: W.(r * (x*w)) = r * (W.(x*w)).  It forms h = silu(g)*u
//    (reference silu.c:75-82, mul_fp32.c) and emits h's digit planes for
//    W_down.
// The dot products are the GEMV's integer digit-plane dots (dot_batch), the
// K-slices of W waves are summed in LDS in a fixed order, so results are
// deterministic.  Compared with RMSNorm-then-GEMV the factor r is applied
// after the product instead of before it (different rounding, same value).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "qh_digits.hpp"
#include "qh_fused.hpp"
#include "qh_vec.hpp"

namespace qh {

constexpr int kBufFlagsF = 0x00020000;  // raw buffer resource word 3 (gfx9 family)
typedef uint32_t v4u32f __attribute__((ext_vector_type(4)));

// RMSNorm scale from per-block sums of squares (each lane sums a strided
// subset in order, then a butterfly; every lane gets the same value).
__device__ __forceinline__ float norm_scale(const float* __restrict__ part, uint32_t nblk, float eps) {
    const int lane = threadIdx.x & 63;
    float s = 0.0f;
    for (uint32_t i = lane; i < nblk; i += 64) s = s + part[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    const float mean = s / (float)(nblk * 32u);
    const float a = mean + eps;
    const float r0 = __builtin_amdgcn_rsqf(a);
    return (r0 * (3.0f - a * (r0 * r0))) * 0.5f;
}

// RESID: one 32-row output block per workgroup, RG row groups of RT rows.
template <int W, int RG, int RT, int J>
__global__ __launch_bounds__(64 * W * RG) void k_gemv_resid(const FusedArgs a) {
    constexpr int TR = RG * RT;
    static_assert(TR == 32, "tile must cover one 32-element output block");
    __shared__ float red[W][TR];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kw = wave % W;
    const int rg = wave / W;
    const uint32_t t = blockIdx.x;
    const uint32_t row_bytes = a.nblk * 20u;

    // ---- this wave's rows ----
    const uint32_t m0 = t * 32u;
    const uint32_t M = a.M[0];
    const uint32_t wrow0 = m0 + (uint32_t)((rg * RT) & 31);

    // ---- weight loads first (they depend on nothing) ----
    uint32_t coff[J];
    bool ok[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t col = (uint32_t)((j * W + kw) * 64 + lane);
        ok[j] = col < a.nblk;
        coff[j] = (ok[j] ? col : 0u) * 20u;
    }
    uint4 q[RT][J];
    float s[RT][J];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const uint32_t row = wrow0 + (uint32_t)r;
        const int nrec = row < M ? (int)row_bytes : 0;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.w[0] + (size_t)row * row_bytes), 0, nrec, kBufFlagsF);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const v4u32f v = __builtin_amdgcn_raw_buffer_load_b128(rs, coff[j], 0, 0);
            q[r][j] = make_uint4(v[0], v[1], v[2], v[3]);
            s[r][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, coff[j] + 16u, 0, 0));
        }
    }
    // ---- epilogue operands of wave 0 (lanes < 32 own the block's rows) ----
    const uint32_t erow = m0 + (uint32_t)(lane & 31);
    float e_res = 0.0f, e_w = 0.0f;
    if (wave == 0) {
        e_res = a.res[erow < M ? erow : 0u];
        e_w = a.wnorm[erow < M ? erow : 0u];
    }
    // ---- input digits and the norm scale ----
    uint4 xp[J][6];
    int kk[J];
    float zz[J];
    {
        uint32_t cols[J];
#pragma unroll
        for (int j = 0; j < J; ++j) cols[j] = coff[j] / 20u;
        load_digits<J>(a.xd, a.pad, cols, ok, xp, kk, zz);
    }

    // ---- dots, per-wave row sums, fixed-order sum over the K-slices ----
    float acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
    // Rows in chunks of up to 8 bound the temporaries of dot_batch.
    constexpr int CH = RT > 8 ? 8 : RT;
#pragma unroll
    for (int r0 = 0; r0 < RT; r0 += CH)
        dot_batch<CH, J>(reinterpret_cast<const uint4(&)[CH][J]>(q[r0]), reinterpret_cast<const float(&)[CH][J]>(s[r0]),
                         xp, kk, zz, ok, reinterpret_cast<float(&)[CH]>(acc[r0]));
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        acc[r] = v;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RT; ++r) red[kw][rg * RT + r] = acc[r];
    }
    __syncthreads();
    if (wave != 0) return;
    float v = 0.0f;
    if (lane < TR) {
        v = red[0][lane];
#pragma unroll
        for (int k2 = 1; k2 < W; ++k2) v += red[k2][lane];
    }
    const bool mine = lane < 32 && erow < M;
    const float xn = e_res + v;
    if (mine) a.y[0][erow] = xn;
    const float u = xn * e_w;
    float sq = mine ? xn * xn : 0.0f;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 32);
    if (lane == 0) a.out_part[m0 / 32u] = sq;
    prep_lane(mine ? u : 0.0f, m0 / 32u, lane < 32, a.pad_out, reinterpret_cast<uint32_t*>(a.xd_out));
}

// Persistent W_gate|W_up + SwiGLU: 8 waves of 8 rows walk 64-row tiles (32
// gate rows + the same 32 up rows).  Each wave's rows are two halves of 4;
// the next half's loads are issued before the current half is computed (a
// one-half-tile pipeline that needs only two 4-row buffers).  Tiles past the
// end read zeros through size-0 buffer resources.
template <int J>
__global__ __launch_bounds__(512) void k_swiglu_p(const FusedArgs a, uint32_t ntiles) {
    constexpr int RH = 4;  // rows per half
    __shared__ float red[64];
    const int lane = threadIdx.x & 63;
    const int rg = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // 0..7, 8 rows each
    const uint32_t sg = (rg >= 4) ? 1u : 0u;
    const uint32_t roff = (uint32_t)((rg * 8) & 31);
    const uint32_t M = a.M[0];
    const uint32_t row_bytes = a.nblk * 20u;
    const uint8_t* __restrict__ wseg = a.w[sg];

    uint32_t coff[J];
    bool ok[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t col = (uint32_t)(j * 64 + lane);
        ok[j] = col < a.nblk;
        coff[j] = (ok[j] ? col : 0u) * 20u;
    }
    // half h of tile t: rows t*32 + roff + 4h .. +3 of this wave's segment
    auto load_half = [&](uint32_t t, int h, uint4 (&q)[RH][J], float (&s)[RH][J]) {
#pragma unroll
        for (int r = 0; r < RH; ++r) {
            const uint32_t row = t * 32u + roff + (uint32_t)(RH * h + r);
            const int nrec = (t < ntiles && row < M) ? (int)row_bytes : 0;
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc((void*)(wseg + (size_t)row * row_bytes), 0, nrec, kBufFlagsF);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const v4u32f v = __builtin_amdgcn_raw_buffer_load_b128(rs, coff[j], 0, 0);
                q[r][j] = make_uint4(v[0], v[1], v[2], v[3]);
                s[r][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, coff[j] + 16u, 0, 0));
            }
        }
    };
    // Both halves of the first tile are requested before the input digits
    // and the norm sums (which the first wait then covers as well); from then
    // on a whole tile is in flight while the current one is computed.
    uint4 qa[RH][J], qb[RH][J];
    float sa[RH][J], sb[RH][J];
    const uint32_t stride = gridDim.x;
    uint32_t t = blockIdx.x;
    load_half(t, 0, qa, sa);
    load_half(t, 1, qb, sb);
    uint4 xp[J][6];
    int kk[J];
    float zz[J];
    {
        uint32_t cols[J];
#pragma unroll
        for (int j = 0; j < J; ++j) cols[j] = coff[j] / 20u;
        load_digits<J>(a.xd, a.pad, cols, ok, xp, kk, zz);
    }
    const float rs_norm = norm_scale(a.in_part, a.nblk, a.eps);
    auto dot_half = [&](const uint4 (&q)[RH][J], const float (&s)[RH][J], float (&out)[RH]) {
        float acc[RH];
#pragma unroll
        for (int r = 0; r < RH; ++r) acc[r] = 0.0f;
        dot_batch<RH, J>(q, s, xp, kk, zz, ok, acc);
#pragma unroll
        for (int r = 0; r < RH; ++r) {
            float v = acc[r];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            out[r] = v;
        }
    };
    auto epilogue = [&](uint32_t t, const float (&v0)[RH], const float (&v1)[RH]) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RH; ++r) {
                red[rg * 8 + r] = v0[r];
                red[rg * 8 + RH + r] = v1[r];
            }
        }
        __syncthreads();
        if (rg == 0) {
            const float gu = rs_norm * red[lane];  // lanes 0..31 gate rows, 32..63 up rows
            const float up = __shfl(gu, (lane & 31) + 32);
            const float hv = silu_approx(gu) * up;
            const bool mine = lane < 32 && t * 32u + (uint32_t)lane < M;
            prep_lane(mine ? hv : 0.0f, t, lane < 32, a.pad_out, reinterpret_cast<uint32_t*>(a.xd_out));
        }
        __syncthreads();  // red[] is reused by the next tile
    };

    while (t < ntiles) {
        float v0[RH], v1[RH];
        dot_half(qa, sa, v0);
        const uint32_t tn = t + stride;
        load_half(tn, 0, qa, sa);
        __builtin_amdgcn_sched_barrier(0);
        dot_half(qb, sb, v1);
        load_half(tn, 1, qb, sb);
        __builtin_amdgcn_sched_barrier(0);
        epilogue(t, v0, v1);
        t = tn;
    }
}

template <int W, int RG, int RT, int J>
static hipError_t run_resid(const FusedArgs& a, uint32_t tiles, hipStream_t s) {
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL((k_gemv_resid<W, RG, RT, J>), dim3(tiles), dim3(64 * W * RG), 0, s, a);
    return hipGetLastError();
}

bool fused_supported(uint32_t nblk) { return nblk >= 1 && nblk <= 128; }

hipError_t launch_fused_resid(FusedArgs a, hipStream_t s) {
    a.nseg = 1;
    if (a.M[0] % 32 != 0 || !a.res || !a.wnorm || !a.xd_out || !a.out_part) return hipErrorInvalidValue;
    const uint32_t tiles = a.M[0] / 32u;
    if (a.nblk <= 64) return run_resid<1, 8, 4, 1>(a, tiles, s);
    if (a.nblk <= 128) return run_resid<1, 8, 4, 2>(a, tiles, s);
    return hipErrorInvalidValue;
}

template <int J>
static hipError_t run_swiglu_p(const FusedArgs& a, uint32_t ntiles, hipStream_t s) {
    static int occ = 0;
    if (occ == 0) {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, k_swiglu_p<J>, 512, 0) != hipSuccess || o < 1) o = 1;
        occ = o;
    }
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu < 1)
        ncu = 256;
    const uint32_t resident = (uint32_t)(occ * ncu);
    const uint32_t grid = ntiles < resident ? ntiles : resident;
    hipLaunchKernelGGL((k_swiglu_p<J>), dim3(grid), dim3(512), 0, s, a, ntiles);
    return hipGetLastError();
}

hipError_t launch_fused_swiglu(FusedArgs a, hipStream_t s) {
    a.nseg = 2;
    if (a.M[0] != a.M[1] || a.M[0] % 32 != 0 || !a.xd_out || !a.in_part) return hipErrorInvalidValue;
    const uint32_t ntiles = a.M[0] / 32u;
    if (ntiles == 0) return hipSuccess;
    if (a.nblk <= 64) return run_swiglu_p<1>(a, ntiles, s);
    if (a.nblk <= 128) return run_swiglu_p<2>(a, ntiles, s);
    return hipErrorInvalidValue;
}

}  // namespace qh
