// k_gemm.hip -- batched Q4_0 x fp32 GEMM for prefill on gfx950 MFMA.
//
// Y[t][m] = sum_k W[m][k] * X[t][k], the per-token GEMV of reference
// src/models/model.c:1120-1561 (every prefill projection loops
// q_gemv_q4_f32_avx2 over the tokens) done as one dense contraction.
//
// Exactness plan (fp32-level accuracy on fp16 matrix cores):
//  * W: the nibble of a Q4_0 element minus 8 is an integer in [-8, 7],
//    exact in fp16.  The block scale s is NOT folded into the operand; each
//    32-element block is one K=32 MFMA step whose fp32 result D is scaled by
//    s in fp32 (inner += s * D), so W enters the matrix core exactly.
//  * X: each token row is scaled by a power of two 2^e (max |x| in
//    [2^14, 2^15)) and split into two fp16 parts: hi = rn(x') and
//    lo = rn(x' - hi) (the subtraction is exact in fp32).  The two parts hold
//    22 significant bits of every element whose lo is an fp16 normal
//    (|x'| >= 2^-3: within 2^17 of the row maximum); smaller elements keep
//    hi's 11 bits plus what the subnormal lo holds (steps of 2^-24).  Two
//    MFMAs per block (hi, lo) against the same weight operand accumulate
//    into one D; the products (q-8)*hi and (q-8)*lo are exact.
//  * Accumulation: a block's D feeds an inner fp32 sum over kInner blocks,
//    which is added to an outer sum (two-level summation): max error
//    relative to sum_k |W x| stays at or below the reference AVX2 order's
//    (four 8-lane accumulators over N/32 blocks) at Llama-3 shapes.
//  * Output: y = outer * 2^-e (exact); a token row with a non-finite input
//    gives NaN outputs (the GEMV kernel's convention).
//
// Tiling: a workgroup of WM x WT waves computes (64*WM rows) x (64*WT
// tokens); each wave a 64x64 tile as 4x4 MFMA 16x16x32 tiles.  K advances
// in steps of 2 blocks staged in LDS (double-buffered, one barrier per
// step): X hi/lo as fp16 rows padded to 144 bytes (conflict-free 16-byte
// reads), W as raw 16-byte nibble blocks + scales, dequantized per lane
// right before the MFMA.  Global loads run ahead of the LDS stages: X one
// step (L2 hits), the weight blocks two steps (HBM latency).  Workgroups are
// ordered so that each XCD keeps one token tile of X resident in its L2 and
// streams the weight rows.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "qh_kernels.hpp"
#include "qh_vec.hpp"

namespace qh {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr int kBufFlagsG = 0x00020000;  // raw buffer resource word 3 (gfx9 family)
constexpr int kKB = 2;                  // Q4_0 blocks per K-step
constexpr int kInner = 16;              // blocks per inner sum

// In-group order of the 8 elements a lane feeds to the MFMA: the nibble
// unpack below yields (e0,e4), (e1,e5), (e2,e6), (e3,e7) as half pairs, so
// position p holds element perm8(p) = {0,4,1,5,2,6,3,7}[p].
__device__ __forceinline__ constexpr int perm8(int p) { return (p >> 1) + 4 * (p & 1); }

// ---------------------------------------------------------------------------
// X preparation: one workgroup per (padded) token row.
// xh/xl: [T_pad][N_pad] fp16 (hi, lo), permuted within groups of 8; columns
// >= N and rows >= T are zero.  meta[t] = (2^-e, non-finite flag).
// The row fed to the matrix cores is one of
//   x                      (plain),
//   (x * r) * norm_w       (RMSNorm, r = rms_scale of the row: the decode
//                           prologue's factor, reference rmsnorm.c:33-89),
//   silu(x) * u            (the SwiGLU product, reference silu.c:75-82 then
//                           mul_fp32.c; x is the gate row, u the up row).
// ---------------------------------------------------------------------------
struct GemmXIn {
    const float* x;
    const float* u;       // SwiGLU mode when non-null
    const float* norm_w;  // RMSNorm mode when non-null
    float eps;
    // Reduction mode when part is non-null: row t is
    // (sum_s part[s][t]) * pmeta[t].x + res[t] (NaN where pmeta[t].y is set),
    // the order of k_gemm_reduce and gemm_store, and is also written to x.
    const float* part;
    uint32_t split;
    const float2* pmeta;
    const float* res;
};

constexpr uint32_t kXpMaxGroups = 16;  // 8-element groups per thread: rows of up to 32768 elements

template <uint32_t kXpGroups>
__global__ __launch_bounds__(256) void k_gemm_xprep(const GemmXIn in, uint32_t T, uint32_t N, uint32_t N_pad,
                                                    _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                    float2* meta) {  // meta may be the producer's pmeta
    __shared__ float red[4];
    __shared__ int red_f[4];
    const uint32_t t = blockIdx.x;
    const bool valid = t < T;  // uniform over the workgroup
    const uint32_t ng = N_pad / 8, nv = valid ? N / 8 : 0u;  // groups of the padded row / holding data
    const float4* x4 = reinterpret_cast<const float4*>(in.x + (size_t)t * N);
    const float4* u4 = in.u ? reinterpret_cast<const float4*>(in.u + (size_t)t * N) : nullptr;
    // The thread's groups g = tid + 256*i, read once (two 16-byte loads each).
    float v[kXpGroups][8];
    float ss = 0.0f;
    // reduction mode: the producer's scale and flag of this row (read before
    // the barriers that precede this kernel's own meta store)
    const float2 pm = (in.part && valid) ? in.pmeta[t] : make_float2(1.0f, 0.0f);
    const size_t pstride = (size_t)T * N / 4;  // float4s per partial plane
#pragma unroll
    for (uint32_t i = 0; i < kXpGroups; ++i) {
        const uint32_t g = threadIdx.x + 256u * i;
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
        if (g < nv) {
            if (in.part) {
                const float4* p4 = reinterpret_cast<const float4*>(in.part + (size_t)t * N);
                a = p4[2 * g];
                b = p4[2 * g + 1];
                uint32_t sp = 1;
                // 4 partials' loads in flight at a time; the sum stays
                // sequential in split order
                for (; sp + 4 <= in.split; sp += 4) {
                    float4 c[4], d[4];
#pragma unroll
                    for (uint32_t u = 0; u < 4; ++u) {
                        c[u] = p4[(sp + u) * pstride + 2 * g];
                        d[u] = p4[(sp + u) * pstride + 2 * g + 1];
                    }
#pragma unroll
                    for (uint32_t u = 0; u < 4; ++u) {
                        a.x += c[u].x; a.y += c[u].y; a.z += c[u].z; a.w += c[u].w;
                        b.x += d[u].x; b.y += d[u].y; b.z += d[u].z; b.w += d[u].w;
                    }
                }
                for (; sp < in.split; ++sp) {
                    const float4 c = p4[sp * pstride + 2 * g], d = p4[sp * pstride + 2 * g + 1];
                    a.x += c.x; a.y += c.y; a.z += c.z; a.w += c.w;
                    b.x += d.x; b.y += d.y; b.z += d.z; b.w += d.w;
                }
                a.x = a.x * pm.x; a.y = a.y * pm.x; a.z = a.z * pm.x; a.w = a.w * pm.x;
                b.x = b.x * pm.x; b.y = b.y * pm.x; b.z = b.z * pm.x; b.w = b.w * pm.x;
                if (in.res) {
                    const float4* r4 = reinterpret_cast<const float4*>(in.res + (size_t)t * N);
                    const float4 c = r4[2 * g], d = r4[2 * g + 1];
                    a.x = c.x + a.x; a.y = c.y + a.y; a.z = c.z + a.z; a.w = c.w + a.w;
                    b.x = d.x + b.x; b.y = d.y + b.y; b.z = d.z + b.z; b.w = d.w + b.w;
                }
                if (pm.y != 0.0f) {
                    const float q = __builtin_nanf("");
                    a = make_float4(q, q, q, q);
                    b = a;
                }
                float4* o4 = reinterpret_cast<float4*>(const_cast<float*>(in.x) + (size_t)t * N);
                o4[2 * g] = a;
                o4[2 * g + 1] = b;
            } else {
                a = x4[2 * g];
                b = x4[2 * g + 1];
            }
        }
        v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
        v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
        if (in.norm_w) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = ss + v[i][e] * v[i][e];
        }
        if (u4 && g < nv) {
            const float4 c = u4[2 * g], d = u4[2 * g + 1];
            const float uu[8] = {c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = silu_approx(v[i][e]) * uu[e];
        }
    }
    if (in.norm_w) {
        // r = newton(rsq(sum/N + eps)), the RMSNorm factor of reference
        // rmsnorm.c:62-71 (the sum in this kernel's fixed order)
        const float sum = block_sum<256>(ss, red);
        const float av = sum / (float)N + in.eps;
        const float r0 = __builtin_amdgcn_rsqf(av);
        const float r = (r0 * (3.0f - av * (r0 * r0))) * 0.5f;
        const float4* w4 = reinterpret_cast<const float4*>(in.norm_w);
#pragma unroll
        for (uint32_t i = 0; i < kXpGroups; ++i) {
            const uint32_t g = threadIdx.x + 256u * i;
            if (g < nv) {
                const float4 c = w4[2 * g], d = w4[2 * g + 1];
                const float ww[8] = {c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) v[i][e] = (v[i][e] * r) * ww[e];
            }
        }
    }
    float m = 0.0f;
    int nf = 0;
#pragma unroll
    for (uint32_t i = 0; i < kXpGroups; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            nf |= !__builtin_isfinite(v[i][e]);
            m = fmaxf(m, fabsf(v[i][e]));
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        nf |= __shfl_xor(nf, off);
    }
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = m;
        red_f[threadIdx.x >> 6] = nf;
    }
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    nf = red_f[0] | red_f[1] | red_f[2] | red_f[3];
    int e = 0;
    if (!nf && m > 0.0f) {
        int E;
        frexpf(m, &E);  // m = f * 2^E, f in [0.5, 1)
        e = 15 - E;     // m * 2^e in [2^14, 2^15)
    }
    _Float16* hr = xh + (size_t)t * N_pad;
    _Float16* lr = xl + (size_t)t * N_pad;
#pragma unroll
    for (uint32_t i = 0; i < kXpGroups; ++i) {
        const uint32_t g = threadIdx.x + 256u * i;
        if (g < ng) {
            h8v hv, lv;
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const float w = nf ? 0.0f : ldexpf(v[i][perm8(p)], e);
                const _Float16 h = (_Float16)w;
                hv[p] = h;
                lv[p] = (_Float16)(w - (float)h);  // the exact difference, rounded
            }
            *reinterpret_cast<h8v*>(hr + g * 8) = hv;
            *reinterpret_cast<h8v*>(lr + g * 8) = lv;
        }
    }
    if (threadIdx.x == 0) meta[t] = make_float2(ldexpf(1.0f, -e), nf ? 1.0f : 0.0f);
}

// ---------------------------------------------------------------------------
// Main kernel
// ---------------------------------------------------------------------------
constexpr int kGemmMaxSeg = 3;

struct GemmArgs {
    const uint8_t* w[kGemmMaxSeg];
    float* y[kGemmMaxSeg];
    const float* res[kGemmMaxSeg];  // optional residual rows added to y (same layout)
    uint32_t M[kGemmMaxSeg];        // weight rows (output columns) of the segment
    uint32_t ld[kGemmMaxSeg];       // row length of y and res (the whole matrix's rows)
    uint32_t mt_end[kGemmMaxSeg];   // cumulative m-tile counts per segment
    uint32_t nseg;
    uint32_t nblk;        // blocks per weight row
    uint32_t T;
    uint32_t N_pad;       // staged X row length (halfs)
    uint32_t n_tt;        // token tiles
    uint32_t split;       // K splits (partials when > 1)
    uint32_t blk_per_split;
    uint32_t xcd_map;     // 1: XCD-aware tile order
    const _Float16* xh;
    const _Float16* xl;   // the low part
    const float2* meta;
    float* part;          // [split][T][M_total-slot] partials (split > 1)
    uint32_t part_ld;     // partial row length (sum of segment M)
    uint32_t part_off[kGemmMaxSeg];  // column offset of each segment in a partial row
};

// Segment of m-tile index mt / of partial-row column c.
__device__ __forceinline__ uint32_t seg_of_tile(const GemmArgs& a, uint32_t mt) {
    return (a.nseg > 1 && mt >= a.mt_end[0] ? 1u : 0u) + (a.nseg > 2 && mt >= a.mt_end[1] ? 1u : 0u);
}
__device__ __forceinline__ uint32_t seg_of_col(const GemmArgs& a, uint32_t c) {
    return (a.nseg > 1 && c >= a.part_off[1] ? 1u : 0u) + (a.nseg > 2 && c >= a.part_off[2] ? 1u : 0u);
}

// Final value of Y[t][m] in segment sg from the fp32 sum v of the scaled
// operands: v * 2^-e, plus the residual when given; NaN for a non-finite row.
__device__ __forceinline__ void gemm_store(const GemmArgs& a, uint32_t sg, uint32_t t, uint32_t m, float v) {
    const float2 mt = a.meta[t];
    const size_t i = (size_t)t * a.ld[sg] + m;
    float y = v * mt.x;
    if (a.res[sg]) y = a.res[sg][i] + y;
    a.y[sg][i] = mt.y != 0.0f ? __builtin_nanf("") : y;
}

// gemm_store of rows m .. m+3 (those below the segment's M), with 16-byte
// accesses where the row length keeps them aligned.
__device__ __forceinline__ void gemm_store4(const GemmArgs& a, uint32_t sg, uint32_t t, uint32_t m, f4v v) {
    const uint32_t M = a.M[sg];
    if ((a.ld[sg] & 3u) != 0 || m + 3 >= M) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (m + r < M) gemm_store(a, sg, t, m + r, v[r]);
        return;
    }
    const float2 mt = a.meta[t];
    const size_t i = (size_t)t * a.ld[sg] + m;
    f4v y = v * mt.x;
    if (a.res[sg]) y = *reinterpret_cast<const f4v*>(a.res[sg] + i) + y;
    if (mt.y != 0.0f) y = f4v{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
    *reinterpret_cast<f4v*>(a.y[sg] + i) = y;
}

// (a & mask) | c in one instruction (the compiler splits it in two when both
// constants are literals).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(c));
    return r;
}

// 8 nibbles of one dword -> 8 fp16 (q - 8), in the perm8 order: half pairs
// (n_c, n_{c+4}) for c = 0..3.  A nibble OR'ed under the fp16 bit pattern of
// 1024 gives 1024 + n (bits 0-3) or 1024 + 16 n (bits 4-7); the first is
// shifted by -1032, the second scaled by 1/16 and shifted by -72 (every step
// exact in fp16).  Nibbles 2, 3, 6, 7 take the same two forms after a shift
// by 8.
__device__ __forceinline__ h8v unpack8(uint32_t w) {
    const uint32_t w8 = w >> 8;
    const h2v lo_shift = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const h2v hi_scale = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2v hi_shift = {(_Float16)-72.0f, (_Float16)-72.0f};
    const h2v p0 = __builtin_bit_cast(h2v, and_or(w, 0x000F000Fu, 0x64006400u)) + lo_shift;
    const h2v p1 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, and_or(w, 0x00F000F0u, 0x64006400u)), hi_scale, hi_shift);
    const h2v p2 = __builtin_bit_cast(h2v, and_or(w8, 0x000F000Fu, 0x64006400u)) + lo_shift;
    const h2v p3 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, and_or(w8, 0x00F000F0u, 0x64006400u)), hi_scale, hi_shift);
    return h8v{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// MI: 16-row weight subtiles per wave, JT: 16-token subtiles per wave (a
// wave's tile is 16*MI x 16*JT; JT < 4 for prompts of a few tokens, whose
// single token tile would otherwise be mostly padding).
template <int WM, int WT, int MI, int JT = 4, int KB = kKB>
__global__ __launch_bounds__(64 * WM * WT) void k_gemm_q4(const GemmArgs a) {
    constexpr int NT = 64 * WM * WT;
    constexpr int WR = 16 * MI;  // weight rows per wave
    constexpr int BM = WR * WM;
    constexpr int BT = 16 * JT * WT;
    constexpr int XCK = 4 * KB;                       // 16-byte X chunks per staged row and part
    constexpr int XROW = 32 * KB + 8;                 // LDS halfs per staged X row (8 pad)
    constexpr int XCH = 2 * XCK * BT / NT;            // 16-byte X chunks per thread per K-step
    constexpr int WBL = (BM * KB + NT - 1) / NT;      // weight blocks per thread per K-step
    constexpr bool kWAll = WBL * NT == BM * KB;       // every thread stages WBL blocks
    static_assert(XCH * NT == 2 * XCK * BT, "tile/thread mismatch");
    static_assert(BM * KB % 64 == 0, "weight staging threads come in whole waves");
    static_assert(KB == 2 || KB == 4, "K-step of 2 or 4 blocks");
    static_assert(kInner % KB == 0, "inner sums end on K-step boundaries");
    // A row's blocks sit in its KB slots rotated by the row, so that the
    // per-lane 16-byte reads of 8 consecutive rows cover all 32 banks.
    constexpr int kSwz = KB == 2 ? 2 : 1;

    __shared__ __attribute__((aligned(16))) _Float16 lx[2][2][BT][XROW];
    __shared__ __attribute__((aligned(16))) uint32_t lw[2][BM][KB][4];
    __shared__ __attribute__((aligned(16))) float ls[2][KB][BM];

    // ---- tile of this workgroup ----
    const uint32_t n_mt = a.mt_end[a.nseg - 1] * a.split;  // (m-tile, split) pairs
    uint32_t mm, tt;
    {
        const uint32_t b = blockIdx.x;
        if (a.xcd_map) {
            const uint32_t xcd = b & 7u, k = b >> 3;
            tt = xcd % a.n_tt;
            mm = xcd / a.n_tt + (8u / a.n_tt) * k;
        } else {
            tt = b % a.n_tt;
            mm = b / a.n_tt;
        }
        if (mm >= n_mt) return;
    }
    const uint32_t mtile = mm / a.split, sp = mm % a.split;
    const uint32_t sg = seg_of_tile(a, mtile);
    const uint32_t m0 = (mtile - (sg ? a.mt_end[sg - 1] : 0u)) * BM;
    const uint32_t t0 = tt * BT;
    const uint32_t M = a.M[sg];
    const uint32_t row_bytes = a.nblk * 20u;
    const uint32_t b_begin = sp * a.blk_per_split;
    const uint32_t b_end = min(a.nblk, b_begin + a.blk_per_split);
    const uint32_t nsteps = b_end > b_begin ? (b_end - b_begin + KB - 1) / KB : 0u;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wt = wave / WM;

    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.w[sg], 0, (int)(M * row_bytes), kBufFlagsG);

    // ---- global -> register staging ----
    // X of step k is loaded one step ahead (it is served by L2); the weight
    // blocks of step k two steps ahead, into register set k & 1, so that
    // their HBM latency has two steps of compute to hide behind.  Within a
    // step the X loads are issued first: the wait before the LDS store then
    // leaves the newest weight loads in flight.
    u4v gx[XCH];
    u4v gq[2][WBL];
    float gs[2][WBL];
    // The thread's X chunks (row t0 + t, 8 halfs at column 8*ch of the step)
    // as pointers fixed for the whole loop.
    const _Float16* xsrc[XCH];
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const uint32_t idx = (uint32_t)(tid + NT * c);
        const uint32_t part = idx / (XCK * BT);
        const uint32_t rem = idx % (XCK * BT);
        const uint32_t t = rem / XCK, ch = rem % XCK;
        xsrc[c] = (part ? a.xl : a.xh) + (size_t)(t0 + t) * a.N_pad + 8u * ch;
    }
    auto load_x = [&](uint32_t step) {
        // < N_pad - (32 KB - 1): splits start on multiples of KB blocks and
        // N_pad is a multiple of 128
        const uint32_t k0 = (b_begin + step * KB) * 32u;
#pragma unroll
        for (int c = 0; c < XCH; ++c) gx[c] = *reinterpret_cast<const u4v*>(xsrc[c] + k0);
    };
    auto load_w = [&](uint32_t step, auto setc) {
        constexpr int set = decltype(setc)::value;
        const uint32_t b0 = b_begin + step * KB;
#pragma unroll
        for (int j = 0; j < WBL; ++j) {
            const uint32_t idx = (uint32_t)(tid + NT * j);
            const uint32_t r = idx / KB, kb = idx % KB;
            const uint32_t b = b0 + kb;
            // rows >= M read zeros; threads past the tile's blocks (kWAll
            // false) load some row of the buffer and store nothing
            const uint32_t off = (m0 + r) * row_bytes + b * 20u;
            // Blocks past the split's end are masked at the LDS store (a
            // select here would wait for the load right away).
            gq[set][j] = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0);
            gs[set][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wrs, off + 16u, 0, 0));
        }
    };
    // LDS buffer `buf` (also the weight register set) <- the staged step.
    auto store_step = [&](uint32_t step, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const uint32_t b0 = b_begin + step * KB;
#pragma unroll
        for (int c = 0; c < XCH; ++c) {
            const uint32_t idx = (uint32_t)(tid + NT * c);
            const uint32_t part = idx / (XCK * BT);
            const uint32_t rem = idx % (XCK * BT);
            const uint32_t t = rem / XCK, ch = rem % XCK;
            *reinterpret_cast<u4v*>(&lx[buf][part][t][8u * ch]) = gx[c];
        }
#pragma unroll
        for (int j = 0; j < WBL; ++j) {
            const uint32_t idx = (uint32_t)(tid + NT * j);
            const uint32_t r = idx / KB, kb = idx % KB;
            if (kWAll || idx < (uint32_t)(BM * KB)) {  // wave-uniform: BM * KB is a multiple of 64
                // A zero scale removes a masked block: its products are finite.
                *reinterpret_cast<u4v*>(&lw[buf][r][kb ^ ((r >> kSwz) & (KB - 1u))][0]) = gq[buf][j];
                ls[buf][kb][r] = b0 + kb < b_end ? gs[buf][j] : 0.0f;
            }
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;

    f4v inner[MI][JT], outer[MI][JT];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            inner[i][j] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
            outer[i][j] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        }

    const int lr = lane & 15, lq = lane >> 4;
    if (nsteps > 0) {
        load_x(0);
        load_w(0, I0{});
        if (nsteps > 1) load_w(1, I1{});
        store_step(0, I0{});
    }
    __syncthreads();
    uint32_t nb_in = 0;  // blocks in the current inner sum
    // One K-step from LDS buffer `buf` (= step & 1).
    auto step_body = [&](uint32_t step, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        using Next = std::integral_constant<int, buf ^ 1>;
        // Issued unconditionally (the last steps reload step nsteps - 1, which
        // is never stored): a load issued on one path only would make the wait
        // before the LDS store cover the newest weight loads as well.
        load_x(min(step + 1, nsteps - 1));
        load_w(min(step + 2, nsteps - 1), bufc);  // set buf held step's weights, now in LDS
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            // The weight fragment is the MFMA's A operand (D rows = weight
            // rows, D columns = tokens): register r of lane l holds weight row
            // 4*(l/16) + r of the subtile for token l%16, so each lane has 4
            // consecutive outputs of one token row, and their 4 scales.
            h8v B[MI];
            f4v s[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int r = WR * wm + 16 * i + lr;
                B[i] = unpack8(lw[buf][r][kb ^ ((r >> kSwz) & (KB - 1))][lq]);
                s[i] = *reinterpret_cast<const f4v*>(&ls[buf][kb][WR * wm + 16 * i + 4 * lq]);
            }
            // One token subtile at a time: its hi and lo parts, then the MI
            // weight subtiles.
#pragma unroll
            for (int j = 0; j < JT; ++j) {
                const int t = 16 * JT * wt + 16 * j + lr;
                const h8v Ah = *reinterpret_cast<const h8v*>(&lx[buf][0][t][32 * kb + 8 * lq]);
                const h8v Al = *reinterpret_cast<const h8v*>(&lx[buf][1][t][32 * kb + 8 * lq]);
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    f4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(B[i], Ah, f4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(B[i], Al, d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) inner[i][j][r] = fmaf(s[i][r], d[r], inner[i][j][r]);
                }
            }
        }
        nb_in += KB;
        if (nb_in >= kInner) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j) {
                    outer[i][j] += inner[i][j];
                    inner[i][j] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
                }
            nb_in = 0;
        }
        if (step + 1 < nsteps) store_step(step + 1, Next{});
        __syncthreads();
    };
    for (uint32_t step = 0; step < nsteps; step += 2) {
        step_body(step, I0{});
        if (step + 1 < nsteps) step_body(step + 1, I1{});
    }

    // ---- epilogue: lane holds weight rows m .. m+3 of token t ----
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const uint32_t m = m0 + WR * wm + 16 * i + 4 * lq;
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const uint32_t t = t0 + 16 * JT * wt + 16 * j + lr;
            const f4v v = outer[i][j] + inner[i][j];
            if (m < M && t < a.T) {
                if (a.split > 1) {
                    float* dst = a.part + ((size_t)sp * a.T + t) * a.part_ld + a.part_off[sg] + m;
                    if ((a.part_ld & 3u) == 0 && (a.part_off[sg] & 3u) == 0 && m + 3 < M) {
                        *reinterpret_cast<f4v*>(dst) = v;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (m + r < M) dst[r] = v[r];
                    }
                } else {
                    gemm_store4(a, sg, t, m, v);
                }
            }
        }
    }
}

// Fixed-order sum of the K-split partials, scaled by 2^-e of the token.
__global__ __launch_bounds__(256) void k_gemm_reduce(const GemmArgs a) {
    const uint32_t ld = a.part_ld;
    const size_t n = (size_t)a.T * ld;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const uint32_t t = (uint32_t)(i / ld), c = (uint32_t)(i % ld);
        float v = a.part[i];
        uint32_t sp = 1;
        // 8 partials' loads in flight at a time; the sum stays sequential
        for (; sp + 8 <= a.split; sp += 8) {
            float w[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) w[u] = a.part[(size_t)(sp + u) * n + i];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) v += w[u];
        }
        for (; sp < a.split; ++sp) v += a.part[(size_t)sp * n + i];
        const uint32_t sg = seg_of_col(a, c);
        gemm_store(a, sg, t, c - a.part_off[sg], v);
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kGemmWM = 4, kGemmWT = 2;
// K-step of the 16- and 32-token tiles: 4 blocks (80 contiguous bytes of
// each weight row per step, half the steps and barriers; their X tile
// leaves the LDS room)
constexpr int kSmallKB = 4;
constexpr uint32_t kGemmBT = 64 * kGemmWT;  // token rows per tile

static uint32_t gemm_tpad(uint32_t T) { return (T + kGemmBT - 1) / kGemmBT * kGemmBT; }
static uint32_t gemm_npad(uint32_t N) { return (N + 127u) & ~127u; }  // whole K-steps of up to 4 blocks

// Launch plan of a GEMM over weight matrices of Ms[0..nseg) rows (each tiled
// on its own), T tokens and nblk blocks per row: the tile height (256 or 192
// rows), the K split (partials plus a reduction pass when > 1; each split
// keeps at least 32 blocks, and at most max_split), and, for whole-K
// launches, a cut: rows from `cut` on (counted over the matrices laid end to
// end) run in 192-row tiles in a second launch.  The cost model is measured
// on MI355X at T = 512: a launch takes rounds x (16 us + K-steps x 2.12 us
// for 256-row tiles, 1.66 us for 192-row tiles), a round being up to 256
// workgroups (one per CU); a reduction about 1 us plus its traffic at 5 TB/s.
// Up to 128 tokens (one 128-token tile) the plan instead takes the smallest
// token tile of 16, 32, 64 or 128 holding them (one wave per token tile
// below 128, 16*JT tokens per wave) and the smallest K split (a power of
// two, each split keeping kInner blocks) that gives at least 224 workgroups
// (448 for the one-wave tiles, of which several fit a CU):
// measured at 16-128 tokens on the Llama-3 shapes, within a few us of the
// best tile and split, 1.2-3.4x faster than 128-token tiles at K split <= 8.
struct GemmPlan {
    uint32_t bm;     // tile height of the (first) launch
    uint32_t split;
    uint32_t cut;    // the total row count: one launch
    uint32_t bt;     // token tile: 128 (two waves of 64 tokens) or 64, 32, 16 (one wave)
};

static uint32_t gemm_rounds(uint32_t wgs) { return (wgs + 255u) / 256u; }

static GemmPlan gemm_plan(const uint32_t* Ms, int nseg, uint32_t T, uint32_t nblk, uint32_t max_split) {
    const uint32_t n_tt = gemm_tpad(T) / kGemmBT;
    uint32_t mtot = 0;
    for (int i = 0; i < nseg; ++i) mtot += Ms[i];
    auto steps_of = [&](uint32_t sp) { return ((nblk + sp - 1) / sp + kKB - 1) / kKB; };
    // m-tiles of rows [r0, r1) of the matrices laid end to end
    auto tiles = [&](uint32_t r0, uint32_t r1, uint32_t bm) {
        uint32_t base = 0, n = 0;
        for (int i = 0; i < nseg; ++i) {
            const uint32_t lo = std::max(r0, base), hi = std::min(r1, base + Ms[i]);
            if (lo < hi) n += (hi - lo + bm - 1) / bm;
            base += Ms[i];
        }
        return n;
    };
    if (T <= kGemmBT) {
        const uint32_t bt = T <= 16u ? 16u : T <= 32u ? 32u : T <= 64u ? 64u : 128u;
        const uint32_t wgs = tiles(0, mtot, 256u) * ((T + bt - 1) / bt);
        uint32_t sp = 1;
        // (each split keeps a whole inner sum of kInner blocks: with shorter
        // splits the sequential sum of the partials can exceed the AVX2
        // order's error at N = 4096)
        // (the small tiles fit two or more workgroups per CU: 448 of them
        // still run in one round)
        const uint32_t target = bt == 128u ? 224u : 448u;
        while (2 * sp <= max_split && wgs * sp < target && nblk >= 2 * sp * kInner) sp *= 2;
        return GemmPlan{256u, sp, mtot, bt};
    }
    max_split = std::min(max_split, 8u);
    auto launch_us = [&](uint32_t wgs, uint32_t bm, uint32_t steps) {
        return gemm_rounds(wgs) * (16.0 + steps * (bm == 256u ? 2.12 : 1.66));
    };
    GemmPlan best{256u, 1u, mtot, kGemmBT};
    double best_c = 1e30;
    for (uint32_t bm : {256u, 192u}) {
        for (uint32_t sp = 1; sp <= max_split; sp *= 2u) {
            if (sp > 1 && nblk / sp < 32u) break;
            double c = launch_us(tiles(0, mtot, bm) * n_tt * sp, bm, steps_of(sp));
            if (sp > 1) c += 1.0 + (double)(sp + 1) * T * mtot * 4.0 / 5e6;
            if (c < best_c) {
                best_c = c;
                best = GemmPlan{bm, sp, mtot, kGemmBT};
            }
        }
    }
    for (uint32_t r = 256u; r < mtot; r += 256u) {
        const double c = launch_us(tiles(0, r, 256u) * n_tt, 256u, steps_of(1)) +
                         launch_us(tiles(r, mtot, 192u) * n_tt, 192u, steps_of(1));
        if (c < best_c) {
            best_c = c;
            best = GemmPlan{256u, 1u, r, kGemmBT};
        }
    }
    return best;
}

// The K split a workspace is sized for: the plan of M_total rows as one
// matrix (a launch over several matrices takes at most this split).
static uint32_t gemm_ws_split(uint32_t M_total, uint32_t T, uint32_t nblk) {
    return gemm_plan(&M_total, 1, T, nblk, 32u).split;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t gemm_workspace_bytes(uint32_t N, uint32_t T, uint32_t M_total) {
    const size_t tp = gemm_tpad(T), np = gemm_npad(N);
    const uint32_t sp = gemm_ws_split(M_total, T, N / 32u);
    size_t b = 2 * align256(tp * np * 2) + align256(tp * 8);
    if (sp > 1) b += align256((size_t)sp * T * M_total * 4);
    return b;
}

// Arguments for rows [r0, r1) of the segments laid end to end, in m-tiles of
// `bm` rows (a range may cut segments: its pieces point into them).
static void gemm_rows_args(GemmArgs& a, const GemmSegs& sg, uint32_t r0, uint32_t r1, uint32_t bm,
                           uint32_t row_bytes) {
    uint32_t base = 0, mt = 0, n = 0;
    for (int i = 0; i < sg.n; ++i) {
        const uint32_t lo = std::max(r0, base), hi = std::min(r1, base + sg.M[i]);
        if (lo < hi) {
            const uint32_t off = lo - base;
            a.w[n] = sg.w[i] + (size_t)off * row_bytes;
            a.y[n] = sg.y[i] + off;
            a.res[n] = sg.res[i] ? sg.res[i] + off : nullptr;
            a.M[n] = hi - lo;
            a.ld[n] = sg.M[i];
            mt += (hi - lo + bm - 1) / bm;
            a.mt_end[n] = mt;
            ++n;
        }
        base += sg.M[i];
    }
    a.nseg = n;
}

hipError_t launch_gemm_ex(const GemmSegs& sg, const GemmRows& in, void* ws, hipStream_t s, GemmDeferred* defer_out) {
    const uint32_t N = in.N, T = in.T;
    const int nseg = sg.n;
    if (defer_out) defer_out->valid = false;
    const GemmDeferred* from = (in.from && in.from->valid) ? in.from : nullptr;
    if (nseg < 1 || nseg > kGemmMaxSeg || T == 0 || N == 0 || N % 32 != 0 || !(in.x || from))
        return hipErrorInvalidValue;
    if (gemm_npad(N) > 8u * 256u * kXpMaxGroups) return hipErrorInvalidValue;  // the row conversion's register tile
    if (in.norm_w && in.u) return hipErrorInvalidValue;
    const uint32_t tp = gemm_tpad(T), np = gemm_npad(N);
    const uint32_t row_bytes = (N / 32u) * 20u;
    uint8_t* p = static_cast<uint8_t*>(ws);
    const size_t plane = align256((size_t)tp * np * 2);
    GemmArgs a{};
    a.xh = reinterpret_cast<_Float16*>(p);
    a.xl = reinterpret_cast<_Float16*>(p + plane);
    a.meta = reinterpret_cast<float2*>(p + 2 * plane);
    float* part = reinterpret_cast<float*>(p + 2 * plane + align256((size_t)tp * 8));
    uint32_t mtot = 0;
    for (int i = 0; i < nseg; ++i) {
        // Weight offsets are 32-bit buffer offsets.
        if (sg.M[i] == 0 || (uint64_t)sg.M[i] * row_bytes >= (1ull << 31)) return hipErrorInvalidValue;
        a.part_off[i] = mtot;
        mtot += sg.M[i];
    }
    const GemmPlan plan = gemm_plan(sg.M, nseg, T, N / 32u, gemm_ws_split(mtot, T, N / 32u));
    a.nblk = N / 32;
    a.T = T;
    a.N_pad = np;
    a.n_tt = (T + plan.bt - 1) / plan.bt;
    a.split = plan.split;
    const uint32_t kb = plan.bt <= 32u ? (uint32_t)kSmallKB : (uint32_t)kKB;  // the kernel's K-step
    a.blk_per_split = ((a.nblk + a.split - 1) / a.split + kb - 1) / kb * kb;
    a.part = part;
    a.part_ld = mtot;
    // The XCD-aware order needs the token-tile count to divide the 8 XCDs.
    a.xcd_map = (8u % a.n_tt == 0) ? 1u : 0u;
    GemmXIn xin{in.x, in.u, in.norm_w, in.eps, nullptr, 0u, nullptr, nullptr};
    if (from) {
        // The producer's partials lie beyond its own staged rows and scales;
        // in a shared workspace this launch's rows and scales must end at or
        // before those (a staged row no longer than the producer's).
        if (!from->y || from->T != T || from->M != N || (from->ws == ws && np > from->n_pad))
            return hipErrorInvalidValue;
        xin.x = from->y;
        xin.part = from->part;
        xin.split = from->split;
        xin.pmeta = from->meta;
        xin.res = from->res;
    }
    // the smallest register tile holding the row: groups of 8 per thread
    const uint32_t per = (np / 8 + 255) / 256;
    auto xprep = per <= 2 ? k_gemm_xprep<2> : per <= 4 ? k_gemm_xprep<4> : per <= 8 ? k_gemm_xprep<8>
                                                                             : k_gemm_xprep<16>;
    // the rows the token tiles read (zeros past T): all tp rows for the
    // 128-token tile, fewer for the small ones
    const uint32_t rows = std::min(tp, a.n_tt * plan.bt);
    hipLaunchKernelGGL(xprep, dim3(rows), dim3(256), 0, s, xin, T, N, np, const_cast<_Float16*>(a.xh),
                       const_cast<_Float16*>(a.xl), const_cast<float2*>(a.meta));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // rows [r0, r1) in tiles of bm rows
    auto launch = [&](uint32_t r0, uint32_t r1, uint32_t bm) -> hipError_t {
        GemmArgs g = a;
        gemm_rows_args(g, sg, r0, r1, bm, row_bytes);
        const uint32_t pairs = g.mt_end[g.nseg - 1] * g.split * g.n_tt;
        const uint32_t grid = g.xcd_map ? (pairs + 7u) / 8u * 8u : pairs;
        if (plan.bt == 16u)
            hipLaunchKernelGGL((k_gemm_q4<kGemmWM, 1, 4, 1, kSmallKB>), dim3(grid), dim3(64 * kGemmWM), 0, s, g);
        else if (plan.bt == 32u)
            hipLaunchKernelGGL((k_gemm_q4<kGemmWM, 1, 4, 2, kSmallKB>), dim3(grid), dim3(64 * kGemmWM), 0, s, g);
        else if (plan.bt == 64u)
            hipLaunchKernelGGL((k_gemm_q4<kGemmWM, 1, 4, 4>), dim3(grid), dim3(64 * kGemmWM), 0, s, g);
        else if (bm == 256u)
            hipLaunchKernelGGL((k_gemm_q4<kGemmWM, kGemmWT, 4>), dim3(grid), dim3(64 * kGemmWM * kGemmWT), 0, s, g);
        else
            hipLaunchKernelGGL((k_gemm_q4<kGemmWM, kGemmWT, 3>), dim3(grid), dim3(64 * kGemmWM * kGemmWT), 0, s, g);
        return hipGetLastError();
    };
    if (plan.cut < mtot) {
        e = launch(0, plan.cut, 256u);
        if (e != hipSuccess) return e;
        return launch(plan.cut, mtot, 192u);
    }
    e = launch(0, mtot, plan.bm);
    if (e != hipSuccess || a.split == 1) return e;
    bool no_res = true;
    for (int i = 0; i < nseg; ++i) no_res = no_res && sg.res[i] == nullptr;
    if (defer_out && (nseg == 1 || no_res) && (mtot & 3u) == 0) {
        // the next GEMM's row conversion sums the partials
        defer_out->valid = true;
        defer_out->part = part;
        defer_out->split = a.split;
        defer_out->T = T;
        defer_out->M = mtot;
        defer_out->meta = a.meta;
        defer_out->res = sg.res[0];
        defer_out->y = nseg == 1 ? sg.y[0] : nullptr;  // several matrices: the consumer knows the layout
        defer_out->ws = ws;
        defer_out->n_pad = np;
        return hipSuccess;
    }
    // the reduction reads the partials by column of the whole row set
    gemm_rows_args(a, sg, 0, mtot, plan.bm, row_bytes);
    const size_t n = (size_t)T * mtot;
    const uint32_t rg = (uint32_t)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_gemm_reduce, dim3(rg), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm(const uint8_t* const* w, float* const* y, const uint32_t* M, int nseg, uint32_t N,
                       const float* X, uint32_t T, void* ws, hipStream_t s) {
    if (nseg < 1 || nseg > kGemmMaxSeg) return hipErrorInvalidValue;
    GemmSegs sg{};
    sg.n = nseg;
    for (int i = 0; i < nseg; ++i) {
        sg.w[i] = w[i];
        sg.y[i] = y[i];
        sg.M[i] = M[i];
    }
    GemmRows in{};
    in.x = X;
    in.T = T;
    in.N = N;
    return launch_gemm_ex(sg, in, ws, s);
}

}  // namespace qh
