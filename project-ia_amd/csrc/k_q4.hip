// k_q4.hip -- Q4_0 kernels for gfx950: bit-exact dequantization, the
// digit-plane preparation of the GEMV input, and the HBM-streaming GEMV.
//
// GEMV design (decode, batch 1, HBM-bound):
//  * x is STATIONARY in VGPRs.  Each lane owns fixed 32-element block
//    columns of W and streams the matching 20-byte blocks of many rows, so x
//    is read once per workgroup instead of once per weight.
//  * The dot product runs on integer dot units.  Per 32-element block of x
//    the prep step picks a power-of-two scale 2^k (|round(x*2^k)| <=
//    7829367, i.e. 23-24 significant bits for the block maximum) and splits
//    the integer into 6 signed 4-bit digit planes.  A weight dword (8
//    nibbles) XOR 0x88888888 is exactly 8 signed 4-bit values (q - 8), so
//    one v_dot8_i32_i4 per plane and dword accumulates sum (q-8)*digit, and
//    Horner over the planes (<<4) yields P = sum_e (q_e - 8) * x_int_e
//    EXACTLY in int32 (|P| <= 32*8*7829367 < 2^31).  The block's
//    contribution is ldexp(s * (float)P, -k).  That is ~37 VALU ops per 32
//    weights instead of ~75 for fp32 unpack + FMA, which keeps the kernel
//    HBM-bound rather than VALU-bound at MI355X bandwidth.
//  * Loads: one global_load_dwordx4 (qs) + one dword (scale) per lane per
//    block; consecutive lanes take consecutive blocks, so each wave-level
//    load covers 1280 contiguous bytes of a row.
//  * Partial sums are reduced across the wave by butterflies and across
//    waves through LDS in a fixed order (deterministic).
// Accuracy (fp64-referenced, relative to sum_j |W_ij x_j|): ~1e-8, below
// the reference AVX2 order's own error at Llama-3 shapes.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "qh_kernels.hpp"
#include "qh_vec.hpp"

namespace qh {

// ---------------------------------------------------------------------------
// Dequantization: reference src/ops/avx2/dequantize.c:25-72.
// off = -8*s; out[e] = fma((float)q_e, s, off); element e in byte e>>1,
// low nibble first.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ blocks,
                                                 float* __restrict__ out, uint64_t n_blocks) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t* p = blocks + b * 20;
    const uint4 q = *reinterpret_cast<const uint4*>(__builtin_assume_aligned(p, 4));
    const float s = *reinterpret_cast<const float*>(__builtin_assume_aligned(p + 16, 4));
    const float off = -8.0f * s;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float4* o = reinterpret_cast<float4*>(out + b * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = fmaf((float)((w[i] >> (4 * j)) & 15u), s, off);
        o[2 * i] = make_float4(v[0], v[1], v[2], v[3]);
        o[2 * i + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

hipError_t launch_dequant(const uint8_t* blocks, float* out, uint64_t n_blocks, hipStream_t s) {
    if (n_blocks == 0) return hipSuccess;
    const uint64_t grid = (n_blocks + 255) / 256;
    hipLaunchKernelGGL(k_dequant, dim3((uint32_t)grid), dim3(256), 0, s, blocks, out, n_blocks);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Digit-plane preparation of one 32-element block.
// ---------------------------------------------------------------------------
constexpr int kDigitMax = 7829367;   // 7 * (16^6 - 1) / 15: largest 6-digit balanced value
constexpr uint32_t kDigitBias = 8947848u;  // 8 * (16^6 - 1) / 15

__device__ inline void prep_block(const float (&v)[32], uint4 (&planes)[6], uint4& meta) {
    float m = 0.0f;
    bool bad = false;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const float a = fabsf(v[e]);
        bad |= !(a <= FLT_MAX);  // NaN or infinity
        m = fmaxf(m, a);
    }
    int k = 0;
    if (!bad && m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m);  // m < 2^E
        k = 23 - E;
        if (rintf(ldexpf(m, k)) > (float)kDigitMax) k -= 1;
    }
    uint32_t pl[6][4];
#pragma unroll
    for (int p = 0; p < 6; ++p)
#pragma unroll
        for (int i = 0; i < 4; ++i) pl[p][i] = 0u;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const int xi = bad ? 0 : (int)rintf(ldexpf(v[e], k));
        const uint32_t u = (uint32_t)(xi + (int)kDigitBias);  // 6 unsigned nibbles = digit + 8
#pragma unroll
        for (int p = 0; p < 6; ++p) pl[p][e >> 3] |= ((u >> (4 * p)) & 15u) << (4 * (e & 7));
    }
#pragma unroll
    for (int p = 0; p < 6; ++p)
        planes[p] = make_uint4(pl[p][0] ^ 0x88888888u, pl[p][1] ^ 0x88888888u,
                               pl[p][2] ^ 0x88888888u, pl[p][3] ^ 0x88888888u);
    const float z = bad ? __builtin_nanf("") : 0.0f;
    meta = make_uint4((uint32_t)k, __float_as_uint(z), 0u, 0u);
}

__device__ inline void store_xd(uint4* __restrict__ xd, uint32_t pad, uint32_t c, const uint4 (&pl)[6],
                                const uint4& meta) {
#pragma unroll
    for (int p = 0; p < 6; ++p) xd[(size_t)p * pad + c] = pl[p];
    xd[(size_t)6 * pad + c] = meta;
}

// Digits of x (no normalisation): one thread per block.
__global__ __launch_bounds__(256) void k_xprep(const float* __restrict__ x, uint32_t nblk, uint32_t pad,
                                               uint4* __restrict__ xd) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= pad) return;
    uint4 pl[6], meta;
    if (c < nblk) {
        float v[32];
        const float4* xp = reinterpret_cast<const float4*>(x + (size_t)c * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 t = xp[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
        prep_block(v, pl, meta);
    } else {
        // Padding columns: all-zero digits (digit 0 is nibble 0) and k = 0.
#pragma unroll
        for (int p = 0; p < 6; ++p) pl[p] = make_uint4(0u, 0u, 0u, 0u);
        meta = make_uint4(0u, 0u, 0u, 0u);
    }
    store_xd(xd, pad, c, pl, meta);
}

// Fused RMSNorm + digits, one workgroup.  RMSNorm follows reference
// src/ops/avx2/rmsnorm.c:33-89 except for the order of the sum of squares
// (a fixed tree here, 8 lane chains there): see rms_scale; h = (x*r)*w.
// Produces the same bits as the standalone RMSNorm kernel.
constexpr int kNormThreads = 1024;

__global__ __launch_bounds__(kNormThreads) void k_norm_xprep(const float* __restrict__ x, uint32_t N,
                                                             const float* __restrict__ w, float eps,
                                                             float* __restrict__ h_out, uint32_t pad,
                                                             uint4* __restrict__ xd) {
    __shared__ float red[kNormThreads / 64];
    const uint32_t tid = threadIdx.x;
    const float r = rms_scale<kNormThreads>(x, N, eps, red);
    const uint32_t nblk = N / 32;
    for (uint32_t c = tid; c < pad; c += kNormThreads) {
        uint4 pl[6], meta;
        if (c < nblk) {
            float v[32];
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const float n = x[(size_t)c * 32 + e] * r;
                v[e] = n * w[(size_t)c * 32 + e];
            }
            if (h_out) {
                float4* hp = reinterpret_cast<float4*>(h_out + (size_t)c * 32);
#pragma unroll
                for (int i = 0; i < 8; ++i) hp[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            }
            prep_block(v, pl, meta);
        } else {
#pragma unroll
            for (int p = 0; p < 6; ++p) pl[p] = make_uint4(0u, 0u, 0u, 0u);
            meta = make_uint4(0u, 0u, 0u, 0u);
        }
        store_xd(xd, pad, c, pl, meta);
    }
}

hipError_t launch_xprep(const float* x, uint32_t N, const float* norm_w, float eps, float* h_out,
                        uint4* xd, hipStream_t s) {
    const uint32_t nblk = N / 32;
    const uint32_t pad = xd_pad(nblk);
    if (norm_w) {
        hipLaunchKernelGGL(k_norm_xprep, dim3(1), dim3(kNormThreads), 0, s, x, N, norm_w, eps, h_out,
                           pad, xd);
    } else {
        hipLaunchKernelGGL(k_xprep, dim3((pad + 255) / 256), dim3(256), 0, s, x, nblk, pad, xd);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
struct GemvArgs {
    const uint8_t* w[4];
    float* y[4];
    const float* res[4];
    uint32_t M[4];
    uint32_t tile_end[4];  // cumulative workgroup counts per segment
    uint32_t nseg;
    uint32_t nblk;
    uint32_t pad;
    const uint4* xd;
};

// Contribution of one block: ldexp(s * P, -k) with P the exact integer dot.
__device__ inline float block_dot(const uint4 q, const float s, const uint4 (&xp)[6], const int k,
                                  const float z) {
    const int w0 = (int)(q.x ^ 0x88888888u), w1 = (int)(q.y ^ 0x88888888u);
    const int w2 = (int)(q.z ^ 0x88888888u), w3 = (int)(q.w ^ 0x88888888u);
    int a = 0;
#pragma unroll
    for (int p = 5; p >= 0; --p) {
        if (p < 5) a <<= 4;
        a = __builtin_amdgcn_sdot8(w0, (int)xp[p].x, a, false);
        a = __builtin_amdgcn_sdot8(w1, (int)xp[p].y, a, false);
        a = __builtin_amdgcn_sdot8(w2, (int)xp[p].z, a, false);
        a = __builtin_amdgcn_sdot8(w3, (int)xp[p].w, a, false);
    }
    const float c = fmaf(s, (float)a, z);
    return ldexpf(c, -k);
}

// W waves split K, G independent row groups per workgroup, RW rows per wave,
// J block columns per lane per K-chunk (K-chunk = 64*W*J blocks).
template <int W, int J, int G, int RW>
__global__ __launch_bounds__(64 * W * G) void k_gemv(const GemvArgs a) {
    constexpr int kChunk = 64 * W * J;
    constexpr int R = 4;  // rows loaded per batch
    static_assert(RW % R == 0, "RW must be a multiple of 4");

    // Segment of this workgroup (uniform).
    const uint32_t t = blockIdx.x;
    uint32_t sg = 0, tbase = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (sg + 1 < a.nseg && t >= a.tile_end[sg]) {
            tbase = a.tile_end[sg];
            ++sg;
        }
    }
    const uint8_t* __restrict__ wseg = a.w[sg];
    const uint32_t M = a.M[sg];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kw = wave % W;
    const int g = wave / W;
    const uint32_t row0 = (t - tbase) * (G * RW) + g * RW;
    const size_t row_bytes = (size_t)a.nblk * 20u;

    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[r] = 0.0f;

    for (uint32_t cb = 0; cb < a.nblk; cb += kChunk) {
        uint4 xp[J][6];
        int kk[J];
        float zz[J];
        uint32_t col[J];
        bool ok[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            col[j] = cb + (uint32_t)((j * W + kw) * 64 + lane);
            ok[j] = col[j] < a.nblk;
            const uint32_t cc = ok[j] ? col[j] : 0u;
#pragma unroll
            for (int p = 0; p < 6; ++p) xp[j][p] = a.xd[(size_t)p * a.pad + cc];
            const uint4 meta = a.xd[(size_t)6 * a.pad + cc];
            kk[j] = (int)meta.x;
            zz[j] = __uint_as_float(meta.y);
        }
#pragma unroll
        for (int rb = 0; rb < RW; rb += R) {
            uint4 q[R][J];
            float s[R][J];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row = row0 + rb + r;
                const uint8_t* rp = wseg + (size_t)row * row_bytes;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    q[r][j] = make_uint4(0u, 0u, 0u, 0u);
                    s[r][j] = 0.0f;
                    if (row < M && ok[j]) {
                        const uint8_t* bp = rp + (size_t)col[j] * 20u;
                        q[r][j] = *reinterpret_cast<const uint4*>(__builtin_assume_aligned(bp, 4));
                        s[r][j] = *reinterpret_cast<const float*>(__builtin_assume_aligned(bp + 16, 4));
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int j = 0; j < J; ++j)
                    if (ok[j]) acc[rb + r] += block_dot(q[r][j], s[r][j], xp[j], kk[j], zz[j]);
        }
    }

    // Reduce each row over the 64 lanes (butterfly: every lane gets the total).
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        acc[r] = v;
    }
    float* __restrict__ y = a.y[sg];
    const float* __restrict__ res = a.res[sg];
    if constexpr (W == 1) {
        if (lane < RW) {
            float v = 0.0f;
#pragma unroll
            for (int r = 0; r < RW; ++r)
                if (r == lane) v = acc[r];
            const uint32_t row = row0 + lane;
            if (row < M) y[row] = res ? res[row] + v : v;
        }
    } else {
        __shared__ float red[G][W][RW];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RW; ++r) red[g][kw][r] = acc[r];
        }
        __syncthreads();
        const int tid = threadIdx.x;
        if (tid < G * RW) {
            const int gg = tid / RW, r = tid % RW;
            float v = red[gg][0][r];
#pragma unroll
            for (int k2 = 1; k2 < W; ++k2) v += red[gg][k2][r];
            const uint32_t row = (t - tbase) * (G * RW) + gg * RW + r;
            if (row < M) y[row] = res ? res[row] + v : v;
        }
    }
}

template <int W, int J, int G, int RW>
static hipError_t run_gemv(const GemvSeg* segs, int nseg, uint32_t nblk, const uint4* xd, hipStream_t s) {
    GemvArgs a{};
    constexpr uint32_t tile_rows = G * RW;
    uint32_t tiles = 0;
    for (int i = 0; i < 4; ++i) {
        if (i < nseg) {
            a.w[i] = segs[i].w;
            a.y[i] = segs[i].y;
            a.res[i] = segs[i].res;
            a.M[i] = segs[i].M;
            tiles += (segs[i].M + tile_rows - 1) / tile_rows;
        }
        a.tile_end[i] = tiles;
    }
    a.nseg = (uint32_t)nseg;
    a.nblk = nblk;
    a.pad = xd_pad(nblk);
    a.xd = xd;
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL((k_gemv<W, J, G, RW>), dim3(tiles), dim3(64 * W * G), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvSeg* segs, int nseg, uint32_t nblk, const uint4* xd, hipStream_t s) {
    if (nseg < 1 || nseg > 4) return hipErrorInvalidValue;
    if (nblk <= 64) return run_gemv<1, 1, 4, 4>(segs, nseg, nblk, xd, s);
    if (nblk <= 128) return run_gemv<1, 2, 4, 4>(segs, nseg, nblk, xd, s);
    if (nblk <= 256) return run_gemv<2, 2, 2, 8>(segs, nseg, nblk, xd, s);
    return run_gemv<4, 2, 1, 16>(segs, nseg, nblk, xd, s);
}

}  // namespace qh
