// k_fused.hip -- the decode step's Q4_0 GEMVs with their neighbours folded
// into prologue and epilogue, so a Llama-3 layer runs as 7 kernels instead
// of 10 (no separate RMSNorm/digit or SwiGLU/digit kernels).
//
// Every workgroup owns one 32-row block of the output vector (64 matrix rows
// for W_gate|W_up: the same 32 rows of both), so the epilogue sees a whole
// 32-element block and can emit the next GEMV's digit planes itself:
//  * RESID  (Wo, W_down): x_new = res + W.x; stores x_new, the digit planes
//    of x_new * w_norm (the next RMSNorm's weight) and the block's sum of
//    squares of x_new.
//  * QKV / LOGITS / SWIGLU consume such an input: the RMSNorm scale
//    r = newton(rsqrt(sum/N + eps)) (reference src/ops/avx2/rmsnorm.c:62-71)
//    comes from the producer's per-block sums (fixed order), and the
//    matrix products are scaled by r: W.(r * (x*w)) = r * (W.(x*w)).
//    QKV then applies RoPE and stores Q and the K/V cache rows; LOGITS stores
//    the logits; SWIGLU forms h = silu(g)*u (reference silu.c:75-82,
//    mul_fp32.c) and emits h's digit planes for W_down.
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

enum : int { kModeQKV = 0, kModeResid = 1, kModeSwiglu = 2, kModeLogits = 3 };

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

template <int W, int RG, int RT, int J, int MODE>
__global__ __launch_bounds__(64 * W * RG) void k_gemv_fused(const FusedArgs a) {
    constexpr int TR = RG * RT;  // rows per tile: 32, or 64 for SWIGLU
    static_assert(MODE == kModeSwiglu ? TR == 64 : TR == 32, "tile must cover one 32-element output block");
    __shared__ float red[W][TR];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kw = wave % W;
    const int rg = wave / W;
    const uint32_t t = blockIdx.x;
    const uint32_t row_bytes = a.nblk * 20u;

    // ---- this wave's rows ----
    uint32_t sg = 0, m0 = 0;
    if (MODE == kModeSwiglu) {
        m0 = t * 32u;
        sg = (rg * RT >= 32) ? 1u : 0u;
    } else {
        uint32_t tbase = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (sg + 1 < a.nseg && t >= a.tile_end[sg]) {
                tbase = a.tile_end[sg];
                ++sg;
            }
        m0 = (t - tbase) * 32u;
    }
    const uint32_t M = a.M[sg];
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
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.w[sg] + (size_t)row * row_bytes), 0, nrec, kBufFlagsF);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const v4u32f v = __builtin_amdgcn_raw_buffer_load_b128(rs, coff[j], 0, 0);
            q[r][j] = make_uint4(v[0], v[1], v[2], v[3]);
            s[r][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, coff[j] + 16u, 0, 0));
        }
    }
    // ---- epilogue operands of wave 0 (lanes < 32 own the block's rows) ----
    const uint32_t erow = m0 + (uint32_t)(lane & 31);
    float e_res = 0.0f, e_w = 0.0f, e_c = 0.0f, e_s = 0.0f;
    uint32_t pos = 0;
    if (wave == 0) {
        if (MODE == kModeResid) {
            e_res = a.res[erow < M ? erow : 0u];
            e_w = a.wnorm[erow < M ? erow : 0u];
        }
        if (MODE == kModeQKV) {
            pos = *a.pos;
            if ((a.rope_mask >> sg) & 1u) {
                const uint32_t hd = a.hd[sg];
                e_c = a.cos_tab[(size_t)pos * hd + erow % hd];
                e_s = a.sin_tab[(size_t)pos * hd + erow % hd];
            }
        }
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
    float rs_norm = 1.0f;
    if (MODE != kModeResid) rs_norm = norm_scale(a.in_part, a.nblk, a.eps);

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

    if (MODE == kModeLogits) {
        if (mine) a.y[0][erow] = rs_norm * v;
    } else if (MODE == kModeQKV) {
        const float vr = rs_norm * v;
        const float pv = __shfl_xor(vr, 1);
        if (mine) {
            float o = vr;
            float* dst = a.y[sg] + erow;
            const uint32_t hd = a.hd[sg];
            if (hd) {
                const uint32_t i = erow % hd;
                if ((a.rope_mask >> sg) & 1u) {
                    // Pair (x0, x1) = (row&~1, row|1): y0 = x0*c - x1*s,
                    // y1 = x1*c + x0*s, products rounded separately.
                    const float t0 = vr * e_c, t1 = pv * e_s;
                    o = (erow & 1u) ? t0 + t1 : t0 - t1;
                }
                dst = a.y[sg] + (size_t)pos * a.pos_stride[sg] + (size_t)(erow / hd) * a.head_stride[sg] + i;
            }
            *dst = o;
        }
    } else if (MODE == kModeResid) {
        const float xn = e_res + v;
        if (mine) a.y[0][erow] = xn;
        const float u = xn * e_w;
        float sq = mine ? xn * xn : 0.0f;
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 32);
        if (lane == 0) a.out_part[m0 / 32u] = sq;
        prep_lane(mine ? u : 0.0f, m0 / 32u, lane < 32, a.pad_out, reinterpret_cast<uint32_t*>(a.xd_out));
    } else {  // kModeSwiglu: lanes 0..31 gate rows, 32..63 up rows
        const float gu = rs_norm * v;
        const float up = __shfl(gu, (lane & 31) + 32);
        const float h = silu_approx(gu) * up;
        prep_lane(mine ? h : 0.0f, m0 / 32u, lane < 32, a.pad_out, reinterpret_cast<uint32_t*>(a.xd_out));
    }
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

template <int W, int RG, int RT, int J, int MODE>
static hipError_t run_fused(const FusedArgs& a, uint32_t tiles, hipStream_t s) {
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL((k_gemv_fused<W, RG, RT, J, MODE>), dim3(tiles), dim3(64 * W * RG), 0, s, a);
    return hipGetLastError();
}

// Shape dispatch by input width: nblk <= 64 (J=1), <= 128 (J=2) on one
// wave per K; up to 448 or 512 blocks (W_down of Llama-3 8B) split over 7
// or 8 waves, each wave all 32 rows of the tile.
template <int MODE>
static hipError_t dispatch(const FusedArgs& a, uint32_t tiles, hipStream_t s) {
    constexpr int RG1 = MODE == kModeSwiglu ? 16 : 8;
    if (a.nblk <= 64) return run_fused<1, RG1, 4, 1, MODE>(a, tiles, s);
    if (a.nblk <= 128) return run_fused<1, RG1, 4, 2, MODE>(a, tiles, s);
    if (MODE == kModeSwiglu) return hipErrorInvalidValue;
    if (a.nblk <= 448) return run_fused<7, 1, 32, 1, MODE == kModeSwiglu ? kModeResid : MODE>(a, tiles, s);
    if (a.nblk <= 512) return run_fused<8, 1, 32, 1, MODE == kModeSwiglu ? kModeResid : MODE>(a, tiles, s);
    return hipErrorInvalidValue;
}

static uint32_t fill_tiles(FusedArgs& a) {
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < 3; ++i) {
        if (i < a.nseg) tiles += (a.M[i] + 31u) / 32u;
        a.tile_end[i] = tiles;
    }
    return tiles;
}

bool fused_supported(uint32_t nblk) { return nblk <= 128 || nblk == 448 || (nblk > 128 && nblk <= 512); }

hipError_t launch_fused_qkv(FusedArgs a, hipStream_t s) {
    if (a.nseg < 1 || a.nseg > 3 || !a.pos) return hipErrorInvalidValue;
    for (uint32_t i = 0; i < a.nseg; ++i)
        if (a.M[i] % 32 != 0 || (a.hd[i] && (a.hd[i] % 32 != 0))) return hipErrorInvalidValue;
    return dispatch<kModeQKV>(a, fill_tiles(a), s);
}

hipError_t launch_fused_resid(FusedArgs a, hipStream_t s) {
    a.nseg = 1;
    if (a.M[0] % 32 != 0 || !a.res || !a.wnorm || !a.xd_out || !a.out_part) return hipErrorInvalidValue;
    return dispatch<kModeResid>(a, fill_tiles(a), s);
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

hipError_t launch_fused_logits(FusedArgs a, hipStream_t s) {
    a.nseg = 1;
    return dispatch<kModeLogits>(a, fill_tiles(a), s);
}

// x = embd[token] (reference model.c:1027-1068) with the first layer's
// RMSNorm input prepared as the RESID epilogue does: digits of x * w_norm
// and per-block sums of squares.  One 32-lane group per block.
__global__ __launch_bounds__(256) void k_embed_prep(const float* __restrict__ embd, const uint32_t* __restrict__ tok,
                                                    uint32_t vocab, uint32_t dim, const float* __restrict__ wnorm,
                                                    float* __restrict__ x, uint32_t pad, uint32_t* __restrict__ xd,
                                                    float* __restrict__ part) {
    uint32_t tk = *tok;
    tk = tk < vocab ? tk : vocab - 1;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const bool valid = i < dim;
    const float xv = valid ? embd[(size_t)tk * dim + i] : 0.0f;
    if (valid) x[i] = xv;
    float sq = xv * xv;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 32);
    if (valid && (i & 31u) == 0) part[i / 32u] = sq;
    prep_lane(valid ? xv * wnorm[i] : 0.0f, i / 32u, valid, pad, xd);
}

hipError_t launch_embed_prep(const float* embd, const uint32_t* tok, uint32_t vocab, uint32_t dim,
                             const float* wnorm, float* x, uint4* xd, float* part, hipStream_t s) {
    if (dim % 32 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed_prep, dim3((dim + 255) / 256), dim3(256), 0, s, embd, tok, vocab, dim, wnorm, x,
                       xd_pad(dim / 32), reinterpret_cast<uint32_t*>(xd), part);
    return hipGetLastError();
}

}  // namespace qh
