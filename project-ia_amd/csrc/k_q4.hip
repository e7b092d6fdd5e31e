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
// Outliers: a block where a few activation outliers set the step (removing
// some 6 of its elements would leave less than 3/64 of its maximum; the
// exact rule is in qh_digits.hpp) also gets a second level of digits for
// the residual x*2^k - x_int, so every element within 2^21 of the block
// maximum is represented exactly; the GEMV adds that level's dot, one plane
// at a time, only in waves whose columns hold such a block (found at the
// barrier that publishes the digits, or with the digits themselves), in a
// loop of its own without prefetch so the level-1 loop keeps its registers
// and occupancy.
// Accuracy (fp64-referenced, relative to sum_j |W_ij x_j|): 0.4-2e-8 at the
// Llama-3 shapes with N(0,1) inputs, at or below the reference AVX2 order's,
// and the same with 1..6 outliers of 1e3..1e5 per block (and mixed sizes)
// meeting zero weights, in one block or in every block (tested).  A block
// left on level 1 keeps at least 3/64 of its maximum outside any 6 of its
// elements; more zero-weighted outliers than that per block (7 or more of
// similar size, next to values 1e3 times smaller) are outside the bound.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "qh_kernels.hpp"
#include "qh_digits.hpp"
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
// Digit planes of the GEMV input.  32 consecutive lanes own one 32-element
// block (lane = element): block max and NaN/Inf flag by cross-lane
// reductions, x_int = round(x * 2^k), its 6 balanced base-16 digits, and the
// 8-lane OR that packs each plane dword.  Lanes 0..5 of each 8-lane group
// store plane dwords, lanes 6..7 of the first group store (k, z).
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;  // 8 blocks per pass

// Digits of x: one lane per element.
__global__ __launch_bounds__(kPrepThreads) void k_xprep(const float* __restrict__ x, uint32_t nblk,
                                                        uint32_t pad, uint32_t* __restrict__ xd) {
    const uint32_t t = blockIdx.x * kPrepThreads + threadIdx.x;
    const uint32_t c = t >> 5;
    const bool valid = c < nblk;
    const float v = valid ? x[t] : 0.0f;
    prep_lane(v, c, valid, pad, xd);
}

// Fused RMSNorm + digits.  Every workgroup computes the same sum of squares
// (identical fixed order, see rms_scale) and prepares its own 8*passes
// blocks.  RMSNorm follows reference src/ops/avx2/rmsnorm.c:33-89 except for
// the order of that sum: h = (x*r)*w, bit-identical to the standalone
// RMSNorm kernel.
constexpr uint32_t kNormPrepBlocksPerWg = 16;

__global__ __launch_bounds__(kPrepThreads) void k_norm_xprep(const float* __restrict__ x, uint32_t N,
                                                             const float* __restrict__ w, float eps,
                                                             float* __restrict__ h_out, uint32_t pad,
                                                             uint32_t* __restrict__ xd) {
    __shared__ float red[kPrepThreads / 64];
    const float r = rms_scale<kPrepThreads>(x, N, eps, red);
    const uint32_t nblk = N / 32;
#pragma unroll
    for (uint32_t pass = 0; pass < kNormPrepBlocksPerWg / (kPrepThreads / 32); ++pass) {
        const uint32_t t = (blockIdx.x * kNormPrepBlocksPerWg + pass * (kPrepThreads / 32)) * 32 + threadIdx.x;
        const uint32_t c = t >> 5;
        const bool valid = c < nblk;
        float v = 0.0f;
        if (valid) {
            const float n = x[t] * r;
            v = n * w[t];
            if (h_out) h_out[t] = v;
        }
        prep_lane(v, c, valid, pad, xd);
    }
}

hipError_t launch_xprep(const float* x, uint32_t N, const float* norm_w, float eps, float* h_out,
                        uint4* xd, hipStream_t s) {
    const uint32_t nblk = N / 32;
    const uint32_t pad = xd_pad(nblk);
    uint32_t* xdw = reinterpret_cast<uint32_t*>(xd);
    if (norm_w) {
        const uint32_t grid = (nblk + kNormPrepBlocksPerWg - 1) / kNormPrepBlocksPerWg;
        hipLaunchKernelGGL(k_norm_xprep, dim3(grid), dim3(kPrepThreads), 0, s, x, N, norm_w, eps, h_out, pad,
                           xdw);
    } else {
        const uint32_t grid = (nblk * 32 + kPrepThreads - 1) / kPrepThreads;
        hipLaunchKernelGGL(k_xprep, dim3(grid), dim3(kPrepThreads), 0, s, x, nblk, pad, xdw);
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
    uint32_t hd[4];        // decode epilogue (0: contiguous store)
    uint32_t head_stride[4];
    uint32_t pos_stride[4];
    uint32_t rope_mask;    // bit i: segment i applies RoPE
    uint32_t nseg;
    uint32_t nblk;
    uint32_t pad;
    const uint4* xd;
    const uint32_t* pos;
    const float* cos_tab;
    const float* sin_tab;
    const float* in_part;  // optional: per-block sums of squares of the un-normalized input
    float eps;             // (row values are then scaled by the RMSNorm factor)
    const float* xf;       // fp32 input (N = 32*nblk) when the kernel makes the digits itself
    const float* xnorm_w;  // with xf: RMSNorm weight; digits of x*w, rows scaled by the norm factor
    float* amax;           // AM: per-workgroup greedy-argmax partials of y, values [0, grid) then
                           // first indices [grid, 2*grid) (as uint32)
};

// Segment of tile t (tiles of `tile_rows` rows, numbered across segments).
__device__ __forceinline__ void seg_of(const GemvArgs& a, uint32_t t, uint32_t& sg, uint32_t& tbase) {
    sg = 0;
    tbase = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (sg + 1 < a.nseg && t >= a.tile_end[sg]) {
            tbase = a.tile_end[sg];
            ++sg;
        }
    }
}

// RMSNorm factor r = newton(rsqrt(sum/N + eps)) (reference rmsnorm.c:62-71)
// from per-block sums of squares: each lane sums a strided subset in order,
// then a butterfly, so every lane of every wave gets the same value.
__device__ __forceinline__ float gemv_norm_scale(const float* __restrict__ part, uint32_t nblk, float eps) {
    const int lane = threadIdx.x & 63;
    float sum = 0.0f;
    for (uint32_t i = lane; i < nblk; i += 64) sum = sum + part[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float mean = sum / (float)(nblk * 32u);
    const float av = mean + eps;
    const float r0 = __builtin_amdgcn_rsqf(av);
    return (r0 * (3.0f - av * (r0 * r0))) * 0.5f;
}

// Raw buffer resource word 3 for gfx9-family parts (32-bit untyped data, no
// swizzle); out-of-range reads return zero.
constexpr int kBufFlags = 0x00020000;
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));

// Store one finished row (value v, RoPE partner pv) of segment sg, with the
// residual rv and the RoPE cos/sin (c, sn) of the row already loaded.  RoPE
// pairs (x0, x1) = (row&~1, row|1): y0 = x0*c - x1*s, y1 = x1*c + x0*s,
// products rounded separately.
__device__ __forceinline__ void store_row_pre(const GemvArgs& a, uint32_t sg, uint32_t row, float v, float pv,
                                              bool odd, uint32_t pos, float rv, float c, float sn) {
    const uint32_t M = a.M[sg];
    if (row >= M) return;
    float* __restrict__ y = a.y[sg];
    const uint32_t hd = a.hd[sg];
    float* dst = y + row;
    if (hd) {
        const uint32_t i = row % hd;
        if ((a.rope_mask >> sg) & 1u) {
            const float t0 = v * c, t1 = pv * sn;
            v = odd ? t0 + t1 : t0 - t1;
        }
        dst = y + (size_t)pos * a.pos_stride[sg] + (size_t)(row / hd) * a.head_stride[sg] + i;
    }
    *dst = a.res[sg] ? rv + v : v;
}

// ---------------------------------------------------------------------------
// Persistent GEMV (input fits one K-chunk: nblk <= 64*W*J).  A "wave group"
// of W waves covers all K columns; it loads its x digits once, then walks
// row tiles of RT rows (tile u, u + stride, ...), loading the next tile's
// blocks while it computes the current one.  A workgroup holds G wave
// groups (G > 1 only with W == 1: the cross-wave reduction of W > 1 needs
// the whole workgroup on one tile).  The grid is sized to what stays
// resident, so there is one wave of workgroups and no per-tile prologue.
// Each tile step costs about one HBM latency (one tile of prefetch), so a
// wave's time follows its number of tiles: splitting rows into smaller,
// evenly balanced pieces adds steps and measured slower.  The weight loads
// keep the default cache policy: the non-temporal hint made this kernel 4-10 %
// slower (a block's 16-byte nibble load and its 4-byte scale load share
// cache lines), although it speeds up plain one-pass 16-byte reads.
// ---------------------------------------------------------------------------
// SW: SwiGLU pair mode (W == 1): tile u holds rows i0..i0+RT/2-1 of w[0]
// (W_gate) followed by the same rows of w[1] (W_up), i0 = u*RT/2, and stores
// h[i] = silu(g_i) * u_i (reference silu.c:75-82, mul_fp32.c) to y[0].
// AM (W == 1, one segment, plain store): every workgroup also writes the
// (largest value, first row holding it) of the rows it stored to a.amax, the
// greedy argmax's partials (arg_better), so no separate pass re-reads y.
template <int W, int J, int G, int RT, bool XF, bool SW = false, bool AM = false>
__global__ __launch_bounds__(64 * W * G) void k_gemv_p(const GemvArgs a) {
    static_assert(W == 1 || G == 1, "multi-wave K split runs one tile per workgroup");
    static_assert(!SW || (W == 1 && RT % 2 == 0), "SwiGLU pairs need one wave per group and even tiles");
    static_assert(!AM || (W == 1 && !SW), "argmax partials are taken in the one-wave store path");
    const int lane = threadIdx.x & 63;
    // The wave index is uniform per wave; readfirstlane makes that visible to
    // the compiler so tile/segment bookkeeping stays scalar (a vector load of
    // a kernel argument would add vmcnt waits that drain the prefetch).
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kw = wave % W;
    const int g = wave / W;
    const uint32_t row_bytes = a.nblk * 20u;
    const uint32_t total = a.tile_end[a.nseg - 1];
    const uint32_t stride = gridDim.x * G;
    // The decode position is read with a vector load issued before the x
    // and weight loads, and turned scalar only where it is used (the RoPE
    // table rows, the KV-cache address): as a scalar load it would join the
    // kernel-argument loads, whose lgkmcnt(0) wait would hold every load of
    // the prologue back by one memory round trip.
    const __amdgpu_buffer_rsrc_t rpos = __builtin_amdgcn_make_buffer_rsrc((void*)a.pos, 0, a.pos ? 4 : 0, kBufFlags);
    const uint32_t pos_v = __builtin_amdgcn_raw_buffer_load_b32(rpos, 0, 0, 0);
    float rs_norm = 1.0f;  // RMSNorm factor: from in_part (after the first tile's loads) or convert_x

    uint32_t coff[J];
    bool ok[J];
    uint4 xp[J][6];
    float am_v = -INFINITY;  // AM: this lane's best stored row so far
    uint32_t am_i = 0xFFFFFFFFu;
    int kk[J];
    float zz[J];
    uint32_t wd[J];  // the columns' wide flags (blocks with level-2 digits)
    uint32_t cols[J];
    // Does the workgroup (fp32 input by lane quads), the wave (wave-local
    // conversion) or, tile by tile, the wave (prepared digits) hold a block
    // that needs level 2?
    bool use_lo = false;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t col = (uint32_t)((j * W + kw) * 64 + lane);
        ok[j] = col < a.nblk;
        cols[j] = ok[j] ? col : 0u;
        coff[j] = cols[j] * 20u;
    }
    // fp32 input: x is loaded with coalesced 16-byte loads before the first
    // tiles' weight loads (so the conversion waits for x only).  Each lane
    // quad of the workgroup converts one block at a time straight from its
    // registers (thread 4c+i: elements 8i..8i+7 of block c) and writes the
    // digit planes to LDS, from which every lane takes its own columns.
    constexpr int kMaxBlk = 64 * J * W;
    constexpr int kThreads = 64 * W * G;
    // One block column per lane and one wave group (J == 1, G == 1): each
    // wave converts exactly the 64 blocks its own lanes consume, one per
    // lane, staged through LDS at a 36-float stride per block (conflict-free
    // 16-byte reads); staging and conversion stay inside the wave (no
    // workgroup barrier, digits go straight to registers).
    constexpr bool kWaveLocal = J == 1 && G == 1;
    constexpr int kQPass = XF ? (4 * kMaxBlk + kThreads - 1) / kThreads : 0;
    constexpr int kLd = XF ? (kWaveLocal ? 8 : 2 * kQPass) : 0;
    constexpr int kXs = 36;
    // LDS: the quad path keeps all 13 planes of every block (levels 1 and 2:
    // level 2 is read per tile when the wave holds a wide block); the
    // wave-local path stages x at kXs floats per block, and each wave then
    // keeps its blocks' level-2 planes in its own part of that staging area
    // (6 * 64 uint4 of its 64 * kXs / 4).
    static_assert(!kWaveLocal || 6 * 64 * 4 <= 64 * kXs, "wave-local level-2 planes must fit the wave's staging");
    constexpr int kLds = !XF ? 1 : (kWaveLocal ? kMaxBlk * kXs / 4 : kXdPlanes * kMaxBlk);
    __shared__ uint4 lds[kLds];
    __shared__ float lds_ss[XF ? W * G : 1];
    __shared__ uint32_t lds_wide[XF ? W * G : 1];  // per wave: converted a wide block
    v4u32 xl[kLd > 0 ? kLd : 1], wl[kLd > 0 ? kLd : 1];
    if constexpr (XF) {
        const __amdgpu_buffer_rsrc_t rx =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.xf, 0, (int)(a.nblk * 128u), kBufFlags);
        const __amdgpu_buffer_rsrc_t rw =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.xnorm_w, 0, a.xnorm_w ? (int)(a.nblk * 128u) : 0, kBufFlags);
#pragma unroll
        for (int i = 0; i < kLd; ++i) {
            const uint32_t f = kWaveLocal ? (uint32_t)(kw * 512 + i * 64 + lane)
                                          : 2u * ((uint32_t)(i >> 1) * kThreads + threadIdx.x) + (uint32_t)(i & 1);
            xl[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, f * 16u, 0, 0);
            wl[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, f * 16u, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    } else {
        load_digits<J>(a.xd, a.pad, cols, ok, xp, kk, zz, wd);
    }
    // x (or x*w with the RMSNorm weight) staged, converted, and the digits
    // of this lane's columns loaded.  RMSNorm: the sum of x^2 is taken per
    // thread over its 16-byte pieces in order, per wave by a butterfly, then
    // over the waves in order, so every wave of every workgroup gets the
    // same factor newton(rsqrt(sum/N + eps)) (reference rmsnorm.c:62-71).
    auto convert_x = [&]() {
        const bool norm = a.xnorm_w != nullptr;
        float ss = 0.0f;
        if constexpr (!kWaveLocal) {
            // Piece i of this thread is elements 8*qi + 4*(i&1) .. +3 of
            // block c of pass i>>1 (thread 4c+qi of the pass); the lane quad
            // of block c converts it straight from registers.
            float xv[kQPass > 0 ? kQPass : 1][8];
#pragma unroll
            for (int i = 0; i < kLd; ++i) {
                float x4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x4[e] = __uint_as_float(xl[i][e]);
                    ss = ss + x4[e] * x4[e];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[i >> 1][4 * (i & 1) + e] = norm ? x4[e] * __uint_as_float(wl[i][e]) : x4[e];
            }
            if (norm) {
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
                if (lane == 0) lds_ss[wave] = ss;
                __syncthreads();
                float tot = lds_ss[0];
#pragma unroll
                for (int i = 1; i < W * G; ++i) tot += lds_ss[i];
                const float av = tot / (float)(a.nblk * 32u) + a.eps;
                const float r0 = __builtin_amdgcn_rsqf(av);
                rs_norm = (r0 * (3.0f - av * (r0 * r0))) * 0.5f;
            }
            uint32_t* ldw = reinterpret_cast<uint32_t*>(lds);
            bool wide_here = false;
            uint32_t kqs[kQPass > 0 ? kQPass : 1];
            int amq[kQPass > 0 ? kQPass : 1];
            bool mq[kQPass > 0 ? kQPass : 1];
            bool any_maybe = false;
#pragma unroll
            for (int ps = 0; ps < kQPass; ++ps) {
                const uint32_t t = (uint32_t)(ps * kThreads) + threadIdx.x;
                const uint32_t c = t >> 2, qi = t & 3u;
                uint32_t pl[6], zq;
                prep_quarter(xv[ps], pl, kqs[ps], zq, amq[ps], mq[ps]);  // whole quads share c, so they agree on c < kMaxBlk
                any_maybe |= mq[ps];
                if (c < (uint32_t)kMaxBlk) {
#pragma unroll
                    for (int p = 0; p < 6; ++p) ldw[((uint32_t)p * kMaxBlk + c) * 4u + qi] = pl[p];
                    ldw[(kXdMeta * kMaxBlk + c) * 4u + qi] = qi == 0 ? kqs[ps] : (qi == 1 ? zq : 0u);
                }
            }
            // Second stage of the wide test, only where a block passed the
            // first (the whole wave takes part: quad sums): the wide word
            // and level 2 of a wide block (the others' level 2 stays
            // unwritten: their readers go by the wide flag).
            if (__ballot(any_maybe) != 0ull) {
#pragma unroll
                for (int ps = 0; ps < kQPass; ++ps) {
                    const uint32_t t = (uint32_t)(ps * kThreads) + threadIdx.x;
                    const uint32_t c = t >> 2, qi = t & 3u;
                    const bool wq = quarter_wide(xv[ps], (int)kqs[ps], amq[ps], mq[ps]);
                    if (wq && c < (uint32_t)kMaxBlk) {
                        if (qi == 2) ldw[(kXdMeta * kMaxBlk + c) * 4u + qi] = 1u;
                        uint32_t pl2[6];
                        prep_quarter_lo(xv[ps], (int)kqs[ps], pl2);
#pragma unroll
                        for (int p = 0; p < 6; ++p) ldw[((kXdLo + (uint32_t)p) * kMaxBlk + c) * 4u + qi] = pl2[p];
                        wide_here = true;
                    }
                }
            }
            // The barrier that publishes the digits also publishes each
            // wave's "converted a wide block" word; every wave ORs them (it
            // reads all or half of the blocks).  The words are read before
            // the digits, so the decision waits for one LDS read only.
            const bool wave_wide = __ballot(wide_here) != 0ull;  // whole wave votes
            if (lane == 0) lds_wide[wave] = wave_wide ? 1u : 0u;
            __syncthreads();
            uint32_t wide_any = 0u;
#pragma unroll
            for (int i = 0; i < W * G; ++i) wide_any |= lds_wide[i];
            use_lo = wide_any != 0u;
#pragma unroll
            for (int j = 0; j < J; ++j) {
#pragma unroll
                for (int p = 0; p < 6; ++p) xp[j][p] = lds[p * kMaxBlk + cols[j]];
                const uint4 m = lds[kXdMeta * kMaxBlk + cols[j]];
                kk[j] = ok[j] ? (int)m.x : 0;
                zz[j] = ok[j] ? __uint_as_float(m.y) : 0.0f;
                wd[j] = ok[j] ? m.z : 0u;
            }
        } else {
            // One block per lane, staged through LDS inside the wave.
            float* xs = reinterpret_cast<float*>(lds);
#pragma unroll
            for (int i = 0; i < kLd; ++i) {
                const uint32_t f = (uint32_t)(kw * 512 + i * 64 + lane);
                v4u32 v = xl[i];
                float x0 = __uint_as_float(v[0]), x1 = __uint_as_float(v[1]);
                float x2 = __uint_as_float(v[2]), x3 = __uint_as_float(v[3]);
                ss = ss + x0 * x0;
                ss = ss + x1 * x1;
                ss = ss + x2 * x2;
                ss = ss + x3 * x3;
                if (norm) {
                    v[0] = __float_as_uint(x0 * __uint_as_float(wl[i][0]));
                    v[1] = __float_as_uint(x1 * __uint_as_float(wl[i][1]));
                    v[2] = __float_as_uint(x2 * __uint_as_float(wl[i][2]));
                    v[3] = __float_as_uint(x3 * __uint_as_float(wl[i][3]));
                }
                if (f < (uint32_t)kMaxBlk * 8u) *reinterpret_cast<v4u32*>(xs + (f >> 3) * kXs + (f & 7u) * 4u) = v;
            }
            // A wave's LDS writes and the reads that follow them are ordered;
            // the norm's cross-wave sum is the only workgroup-wide step (norm
            // is uniform).
            if (norm) {
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
                if (lane == 0) lds_ss[wave] = ss;
                __syncthreads();
                float tot = lds_ss[0];
#pragma unroll
                for (int i = 1; i < W * G; ++i) tot += lds_ss[i];
                const float av = tot / (float)(a.nblk * 32u) + a.eps;
                const float r0 = __builtin_amdgcn_rsqf(av);
                rs_norm = (r0 * (3.0f - av * (r0 * r0))) * 0.5f;
            }
            float xw[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const v4u32 v = *reinterpret_cast<const v4u32*>(xs + (uint32_t)(kw * 64 + lane) * kXs + (uint32_t)i * 4u);
                xw[4 * i] = __uint_as_float(v[0]);
                xw[4 * i + 1] = __uint_as_float(v[1]);
                xw[4 * i + 2] = __uint_as_float(v[2]);
                xw[4 * i + 3] = __uint_as_float(v[3]);
            }
            uint4 o[13];
            prep_block(xw, o);
#pragma unroll
            for (int p = 0; p < 6; ++p) xp[0][p] = o[p];
            kk[0] = ok[0] ? (int)o[kXdMeta].x : 0;
            zz[0] = ok[0] ? __uint_as_float(o[kXdMeta].y) : 0.0f;
            wd[0] = ok[0] ? o[kXdMeta].z : 0u;
            use_lo = __ballot(wd[0] != 0u) != 0ull;
            // Level-2 planes into this wave's own staging rows, which this
            // lane's reads above have already consumed (a wave's LDS
            // operations complete in order).
            if (wd[0]) {
                uint4* lo2 = reinterpret_cast<uint4*>(xs + (uint32_t)(kw * 64) * kXs);
#pragma unroll
                for (int p = 0; p < 6; ++p) lo2[p * 64 + lane] = o[kXdLo + p];
            }
        }
    };

    // Row r of a tile is read through a buffer resource whose base is the
    // row and whose size is the row's bytes (0 past the last row): the
    // per-lane column offsets stay fixed for the whole kernel, the row base
    // lives in scalar registers, and out-of-range rows, columns and tiles
    // read zeros (a zero scale) without touching memory.  Every load is
    // therefore unconditional, and the epilogue's operands (residual,
    // RoPE cos/sin of the row a lane stores) are loaded with the tile: an
    // epilogue load, or a prefetch under a branch, would make the in-order
    // vmcnt wait drain the next tile's loads.
    struct Epi {
        float res, c, sn;
    };
    auto load_tile = [&](uint32_t u, uint4 (&q)[RT][J], float (&s)[RT][J], Epi& e) {
        if constexpr (SW) {
            const uint32_t M = a.M[0], i0 = u * (uint32_t)(RT / 2);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const uint32_t row = i0 + (uint32_t)(r % (RT / 2));
                const int nrec = row < M ? (int)row_bytes : 0;
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    (void*)(a.w[r < RT / 2 ? 0 : 1] + (size_t)row * row_bytes), 0, nrec, kBufFlags);
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(rs, coff[j], 0, 0);
                    q[r][j] = make_uint4(v[0], v[1], v[2], v[3]);
                    s[r][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, coff[j] + 16u, 0, 0));
                }
            }
            e.res = e.c = e.sn = 0.0f;
            return;
        }
        uint32_t sg, tbase;
        seg_of(a, u, sg, tbase);
        const uint8_t* __restrict__ wseg = a.w[sg];
        const uint32_t M = a.M[sg];
        const uint32_t row0 = (u - tbase) * RT;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint32_t row = row0 + (uint32_t)r;
            const int nrec = row < M ? (int)row_bytes : 0;
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc((void*)(wseg + (size_t)row * row_bytes), 0, nrec, kBufFlags);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(rs, coff[j], 0, 0);
                q[r][j] = make_uint4(v[0], v[1], v[2], v[3]);
                s[r][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, coff[j] + 16u, 0, 0));
            }
        }
        const uint32_t erow = row0 + (uint32_t)(lane & (RT - 1));
        const float* res = a.res[sg];
        const __amdgpu_buffer_rsrc_t rr =
            __builtin_amdgcn_make_buffer_rsrc((void*)res, 0, res ? (int)(M * 4u) : 0, kBufFlags);
        e.res = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr, erow * 4u, 0, 0));
        const uint32_t hd = a.hd[sg];
        const bool rope = (a.rope_mask >> sg) & 1u;
        const uint32_t hdr = rope ? hd : 0u;
        const uint32_t pos = __builtin_amdgcn_readfirstlane(pos_v);
        const uint32_t i = rope ? erow % hd : 0u;
        const __amdgpu_buffer_rsrc_t rc =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.cos_tab + (size_t)pos * hdr), 0, (int)(hdr * 4u), kBufFlags);
        const __amdgpu_buffer_rsrc_t rn =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.sin_tab + (size_t)pos * hdr), 0, (int)(hdr * 4u), kBufFlags);
        e.c = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, i * 4u, 0, 0));
        e.sn = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rn, i * 4u, 0, 0));
    };

    // Level-2 plane p of this lane's column j: from LDS (fp32 input) or from
    // the prepared digits in HBM.
    auto lo_plane = [&](int j, int p, uint32_t salt) -> uint4 {
        if constexpr (XF) {
            if constexpr (kWaveLocal) {
                const uint4* w2 = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(lds) +
                                                                 (uint32_t)(kw * 64) * kXs) + (lane + salt);
                return w2[p * 64];
            } else {
                return (lds + (cols[j] + salt))[(kXdLo + (uint32_t)p) * kMaxBlk];
            }
        } else {
            return load_lo_plane(a.xd, a.pad, cols[j], ok[j], p, salt);
        }
    };
    // Cross-wave partial sums of a tile (W > 1).  Declared here, not in the
    // lambda below: each instantiation of a generic lambda would get its own
    // array, and waves of one workgroup may run different instantiations.
    __shared__ float red[W > 1 ? W : 1][RT];

    // lo2: std::true_type for the level-1 + level-2 dot, std::false_type for
    // level 1 alone.
    auto finish_tile = [&](auto lo2, uint32_t u, const uint4 (&q)[RT][J], const float (&s)[RT][J], const Epi& e) {
        float acc[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
        if constexpr (std::is_same_v<decltype(lo2), std::true_type>) {
            dot_batch2<RT, J>(q, s, xp, lo_plane, kk, zz, ok, wd, acc);
        } else {
            dot_batch<RT, J>(q, s, xp, kk, zz, ok, acc);
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            float v = acc[r];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            acc[r] = v * rs_norm;
        }
        if constexpr (SW) {
            const uint32_t i = u * (uint32_t)(RT / 2) + (uint32_t)lane;
            if (lane < RT / 2 && i < a.M[0]) {
                float g = acc[0], up = acc[RT / 2];
#pragma unroll
                for (int r = 1; r < RT / 2; ++r) {
                    g = (r == lane) ? acc[r] : g;
                    up = (r == lane) ? acc[r + RT / 2] : up;
                }
                a.y[0][i] = silu_approx(g) * up;
            }
            return;
        }
        uint32_t sg, tbase;
        seg_of(a, u, sg, tbase);
        const uint32_t row0 = (u - tbase) * RT;
        const uint32_t pos = __builtin_amdgcn_readfirstlane(pos_v);
        if constexpr (W == 1) {
            if (lane < RT) {
                float v = acc[0], pv = acc[1];
#pragma unroll
                for (int r = 1; r < RT; ++r) v = (r == lane) ? acc[r] : v;
#pragma unroll
                for (int r = 0; r < RT; ++r) pv = (r == (lane ^ 1)) ? acc[r] : pv;
                store_row_pre(a, sg, row0 + lane, v, pv, lane & 1, pos, e.res, e.c, e.sn);
                if constexpr (AM) {
                    const uint32_t row = row0 + (uint32_t)lane;
                    if (row < a.M[sg] && arg_better(v, row, am_v, am_i)) {
                        am_v = v;
                        am_i = row;
                    }
                }
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < RT; ++r) red[kw][r] = acc[r];
            }
            __syncthreads();
            if ((int)threadIdx.x < RT) {
                const int r = threadIdx.x;
                float v = red[0][r], pv = red[0][r ^ 1];
#pragma unroll
                for (int k2 = 1; k2 < W; ++k2) {
                    v += red[k2][r];
                    pv += red[k2][r ^ 1];
                }
                store_row_pre(a, sg, row0 + r, v, pv, r & 1, pos, e.res, e.c, e.sn);
            }
            __syncthreads();  // red[] is reused by the next tile
        }
    };

    uint4 qa[RT][J], qb[RT][J];
    float sa[RT][J], sb[RT][J];
    Epi ea, eb;
    uint32_t u = blockIdx.x * G + g;
    load_tile(u, qa, sa, ea);
    if constexpr (XF) {
        __builtin_amdgcn_sched_barrier(0);
        convert_x();
    } else if (a.in_part) {
        __builtin_amdgcn_sched_barrier(0);
        rs_norm = gemv_norm_scale(a.in_part, a.nblk, a.eps);
    }
    // Level 1 + 2, one tile at a time: no prefetch, so the level-2
    // registers fit in those of a prefetched tile and the kernel keeps the
    // occupancy of the level-1 loop.
    auto level2_loop = [&]() {
        while (u < total) {
            finish_tile(std::true_type{}, u, qa, sa, ea);
            u += stride;
            if (u >= total) break;
            load_tile(u, qa, sa, ea);
        }
    };
    // Level 1, double-buffered: qa holds tile u; each half step issues the
    // next tile's loads, then the scheduling barrier keeps them ahead of any
    // instruction that waits on the current tile's data.  (Two tiles of
    // prefetch measured slower: more concurrent row streams; so did a loop
    // entered with the next tile already issued.)
    auto level1_loop = [&]() {
        while (u < total) {
            uint32_t un = u + stride;
            load_tile(un, qb, sb, eb);
            __builtin_amdgcn_sched_barrier(0);
            finish_tile(std::false_type{}, u, qa, sa, ea);
            u = un;
            if (u >= total) break;
            un = u + stride;
            load_tile(un, qa, sa, ea);
            __builtin_amdgcn_sched_barrier(0);
            finish_tile(std::false_type{}, u, qb, sb, eb);
            u = un;
        }
    };
    if constexpr (XF) {
        // The conversion has already set use_lo (no wait on memory).
        if (use_lo)
            level2_loop();
        else
            level1_loop();
    } else {
        // Prepared digits: the wide flags arrive with the digits, so the
        // second tile's loads go out before waiting on them (a level-2 run
        // drops that tile and loads it again), and the first step of the
        // level-1 loop is peeled.  With waves splitting K the choice is made
        // workgroup-uniform (the cross-wave reduction has barriers in it);
        // not a decode-step shape.
        if (u < total) {
            uint32_t un = u + stride;
            load_tile(un, qb, sb, eb);
            __builtin_amdgcn_sched_barrier(0);
            bool any = false;
#pragma unroll
            for (int j = 0; j < J; ++j) any = any || (ok[j] && wd[j] != 0u);
            if constexpr (W > 1)
                use_lo = __syncthreads_or(any) != 0;
            else
                use_lo = __ballot(any) != 0ull;
            if (use_lo) {
                level2_loop();
            } else {
                finish_tile(std::false_type{}, u, qa, sa, ea);
                u = un;
                if (u < total) {
                    un = u + stride;
                    load_tile(un, qa, sa, ea);
                    __builtin_amdgcn_sched_barrier(0);
                    finish_tile(std::false_type{}, u, qb, sb, eb);
                    u = un;
                    level1_loop();
                }
            }
        }
    }
    if constexpr (AM) {
        // Every wave reaches this point (the loop only breaks).
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(am_v, off);
            const uint32_t oi = (uint32_t)__shfl_xor((int)am_i, off);
            if (arg_better(ov, oi, am_v, am_i)) {
                am_v = ov;
                am_i = oi;
            }
        }
        __shared__ float am_sv[G];
        __shared__ uint32_t am_si[G];
        if (lane == 0) {
            am_sv[g] = am_v;
            am_si[g] = am_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
            for (int k = 1; k < G; ++k)
                if (arg_better(am_sv[k], am_si[k], am_v, am_i)) {
                    am_v = am_sv[k];
                    am_i = am_si[k];
                }
            a.amax[blockIdx.x] = am_v;
            reinterpret_cast<uint32_t*>(a.amax)[gridDim.x + blockIdx.x] = am_i;
        }
    }
}

// W waves split K, G independent row groups per workgroup, RW rows per wave
// (processed R at a time, the next batch loaded while the current one is
// computed), J block columns per lane per K-chunk (K-chunk = 64*W*J blocks).
// Every load is unconditional: out-of-range rows/columns read a clamped,
// in-bounds address and are masked (scale and digits zeroed), so the
// compiler keeps all loads of a batch in flight together.
template <int W, int J, int G, int RW, int R>
__global__ __launch_bounds__(64 * W * G) void k_gemv(const GemvArgs a) {
    constexpr int kChunk = 64 * W * J;
    constexpr int NB = RW / R;
    static_assert(RW % R == 0, "RW must be a multiple of R");

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
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kw = wave % W;
    const int g = wave / W;
    const uint32_t row0 = (t - tbase) * (G * RW) + g * RW;
    const size_t row_bytes = (size_t)a.nblk * 20u;

    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[r] = 0.0f;

    for (uint32_t cb = 0; cb < a.nblk; cb += kChunk) {
        uint32_t coff[J];
        bool ok[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t col = cb + (uint32_t)((j * W + kw) * 64 + lane);
            ok[j] = col < a.nblk;
            coff[j] = (ok[j] ? col : 0u) * 20u;
        }
        uint4 q[2][R][J];
        float s[2][R][J];
        auto load_batch = [&](int b, int buf) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t row = row0 + (uint32_t)(b * R + r);
                row = row < M ? row : M - 1u;
                const uint8_t* rp = wseg + (size_t)row * row_bytes;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint8_t* bp = rp + coff[j];
                    q[buf][r][j] = *reinterpret_cast<const uint4*>(__builtin_assume_aligned(bp, 4));
                    s[buf][r][j] = *reinterpret_cast<const float*>(__builtin_assume_aligned(bp + 16, 4));
                }
            }
        };
        load_batch(0, 0);

        uint4 xp[J][6];
        int kk[J];
        float zz[J];
        uint32_t cols[J];
        uint32_t wd[J];
        bool any = false;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t cc = coff[j] / 20u;
            cols[j] = cc;
#pragma unroll
            for (int p = 0; p < 6; ++p) {
                const uint4 v = a.xd[(size_t)p * a.pad + cc];
                xp[j][p] = ok[j] ? v : make_uint4(0u, 0u, 0u, 0u);
            }
            const uint4 meta = a.xd[(size_t)kXdMeta * a.pad + cc];
            kk[j] = ok[j] ? (int)meta.x : 0;
            zz[j] = ok[j] ? __uint_as_float(meta.y) : 0.0f;
            wd[j] = ok[j] ? meta.z : 0u;
            any = any || wd[j] != 0u;
        }
        const bool wave_wide = __ballot(any) != 0ull;
        auto lo_plane = [&](int j, int p, uint32_t salt) -> uint4 {
            return load_lo_plane(a.xd, a.pad, cols[j], ok[j], p, salt);
        };

        if (wave_wide) {
            // Level 1 + 2, one batch at a time (no prefetch: the level-2
            // registers fit in those of the prefetched batch).
            static_assert(R % 2 == 0, "the level-2 path runs rows in pairs");
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b > 0) load_batch(b, 0);
#pragma unroll
                for (int h = 0; h < R / 2; ++h) {
                    uint4 qh[2][J];
                    float sh[2][J], part[2];
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
#pragma unroll
                        for (int j = 0; j < J; ++j) {
                            qh[r][j] = q[0][2 * h + r][j];
                            sh[r][j] = s[0][2 * h + r][j];
                        }
                        part[r] = acc[b * R + 2 * h + r];
                    }
                    dot_batch2<2, J>(qh, sh, xp, lo_plane, kk, zz, ok, wd, part);
#pragma unroll
                    for (int r = 0; r < 2; ++r) acc[b * R + 2 * h + r] = part[r];
                }
            }
        } else {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b + 1 < NB) load_batch(b + 1, (b + 1) & 1);
                float part[R];
#pragma unroll
                for (int r = 0; r < R; ++r) part[r] = acc[b * R + r];
                dot_batch<R, J>(q[b & 1], s[b & 1], xp, kk, zz, ok, part);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[b * R + r] = part[r];
            }
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
            float v = acc[0], pv = acc[1];
#pragma unroll
            for (int r = 1; r < RW; ++r) v = (r == lane) ? acc[r] : v;
#pragma unroll
            for (int r = 0; r < RW; ++r) pv = (r == (lane ^ 1)) ? acc[r] : pv;
            const uint32_t row = row0 + lane;
            const uint32_t hd = a.hd[sg];
            float* dst = y + row;
            if (hd) {
                const uint32_t pos = *a.pos;
                const uint32_t i = row % hd;
                if ((a.rope_mask >> sg) & 1u) {
                    // Pair (x0, x1) = (row&~1, row|1): y0 = x0*c - x1*s,
                    // y1 = x1*c + x0*s, products rounded separately.
                    const float c = a.cos_tab[(size_t)pos * hd + i];
                    const float sn = a.sin_tab[(size_t)pos * hd + i];
                    const float t0 = v * c, t1 = pv * sn;
                    v = (lane & 1) ? t0 + t1 : t0 - t1;
                }
                dst = y + (size_t)pos * a.pos_stride[sg] + (size_t)(row / hd) * a.head_stride[sg] + i;
            }
            if (row < M) *dst = res ? res[row] + v : v;
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

template <int W, int J, int G, int RW, int R>
static hipError_t run_gemv(const GemvSeg* segs, int nseg, uint32_t nblk, const uint4* xd, hipStream_t s,
                           const GemvDecode* dec) {
    GemvArgs a{};
    constexpr uint32_t tile_rows = G * RW;
    uint32_t tiles = 0;
    for (int i = 0; i < 4; ++i) {
        if (i < nseg) {
            a.w[i] = segs[i].w;
            a.y[i] = segs[i].y;
            a.res[i] = segs[i].res;
            a.M[i] = segs[i].M;
            a.hd[i] = segs[i].hd;
            a.head_stride[i] = segs[i].head_stride;
            a.pos_stride[i] = segs[i].pos_stride;
            if (segs[i].rope) a.rope_mask |= 1u << i;
            // The decode epilogue exists on the single-wave-per-row path only,
            // and RoPE needs whole pairs inside one wave's rows.
            if (segs[i].hd && (W != 1 || !dec || !dec->pos || (segs[i].hd % 2) != 0)) return hipErrorInvalidValue;
            if (segs[i].rope && (!dec->cos_tab || !dec->sin_tab || (RW % 2) != 0)) return hipErrorInvalidValue;
            tiles += (segs[i].M + tile_rows - 1) / tile_rows;
        }
        a.tile_end[i] = tiles;
    }
    a.nseg = (uint32_t)nseg;
    a.nblk = nblk;
    a.pad = xd_pad(nblk);
    a.xd = xd;
    if (dec) {
        a.pos = dec->pos;
        a.cos_tab = dec->cos_tab;
        a.sin_tab = dec->sin_tab;
        if (dec->in_part) return hipErrorInvalidValue;  // norm scale: persistent kernel only
    }
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL((k_gemv<W, J, G, RW, R>), dim3(tiles), dim3(64 * W * G), 0, s, a);
    return hipGetLastError();
}

static int g_num_cu = 0;

static int num_cu() {
    if (g_num_cu == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_num_cu = n;
        else
            g_num_cu = 256;
    }
    return g_num_cu;
}

// Persistent grid: as many groups of G tiles as are resident at once, with
// the one-wave shapes limited to 2 or 3 workgroups per CU.
constexpr int kOneWaveShortWgPerCu = 2;
constexpr int kOneWaveLongWgPerCu = 3;

template <int W, int J, int G, int RT, bool XF, bool SW = false, bool AM = false>
static uint32_t gemv_p_grid(uint32_t tiles) {
    static int occ = 0;
    if (occ == 0) {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, k_gemv_p<W, J, G, RT, XF, SW, AM>, 64 * W * G, 0) !=
                hipSuccess ||
            o < 1)
            o = 1;
        occ = o;
    }
    // One-wave launches run fewer workgroups per CU than their registers
    // allow (3 or 4): fewer concurrent row streams are faster.  Measured:
    // launches of at most two tiles per wave at full occupancy (Q|K|V, Wo)
    // and the pair-mode W_gate|W_up at 2 per CU (Q|K|V 7.0 -> 6.2 us; decode
    // 521 -> 544 tok/s; 1 per CU is slower); longer launches at 3 (the
    // 2-segment W_gate|W_up 16.5 us at 2 per CU, 15.65 us at 3).  The LM
    // head with argmax partials keeps its full occupancy.
    const uint32_t full_waves = (uint32_t)(occ * num_cu() * G);
    const int cap = (SW || tiles <= 2u * full_waves) ? kOneWaveShortWgPerCu : kOneWaveLongWgPerCu;
    const int per_cu = (W == 1 && !AM && occ > cap) ? cap : occ;
    const uint32_t groups = (tiles + G - 1) / G;
    const uint32_t resident = (uint32_t)(per_cu * num_cu());
    return groups < resident ? groups : resident;
}

template <int W, int J, int G, int RT, bool XF, bool SW = false, bool AM = false>
static hipError_t launch_gemv_p(const GemvArgs& a, uint32_t tiles, hipStream_t s) {
    const uint32_t grid = gemv_p_grid<W, J, G, RT, XF, SW, AM>(tiles);
    hipLaunchKernelGGL((k_gemv_p<W, J, G, RT, XF, SW, AM>), dim3(grid), dim3(64 * W * G), 0, s, a);
    return hipGetLastError();
}

// xd: prepared digit planes, or xf: the fp32 input (converted in-kernel).
template <int W, int J, int G, int RT>
static hipError_t run_gemv_p(const GemvSeg* segs, int nseg, uint32_t nblk, const uint4* xd, const float* xf,
                             hipStream_t s, const GemvDecode* dec) {
    GemvArgs a{};
    uint32_t tiles = 0;
    for (int i = 0; i < 4; ++i) {
        if (i < nseg) {
            a.w[i] = segs[i].w;
            a.y[i] = segs[i].y;
            a.res[i] = segs[i].res;
            a.M[i] = segs[i].M;
            a.hd[i] = segs[i].hd;
            a.head_stride[i] = segs[i].head_stride;
            a.pos_stride[i] = segs[i].pos_stride;
            if (segs[i].rope) a.rope_mask |= 1u << i;
            if (segs[i].hd && (!dec || !dec->pos || (segs[i].hd % 2) != 0)) return hipErrorInvalidValue;
            if (segs[i].rope && (!dec->cos_tab || !dec->sin_tab || (RT % 2) != 0)) return hipErrorInvalidValue;
            tiles += (segs[i].M + RT - 1) / RT;
        }
        a.tile_end[i] = tiles;
    }
    a.nseg = (uint32_t)nseg;
    a.nblk = nblk;
    a.pad = xd_pad(nblk);
    a.xd = xd;
    if (dec) {
        a.pos = dec->pos;
        a.cos_tab = dec->cos_tab;
        a.sin_tab = dec->sin_tab;
        a.in_part = dec->in_part;
        a.eps = dec->eps;
    }
    a.xf = xf;
    a.xnorm_w = (xf && dec) ? dec->norm_w : nullptr;
    if (tiles == 0) return hipSuccess;
    if (xf) return launch_gemv_p<W, J, G, RT, true>(a, tiles, s);
    return launch_gemv_p<W, J, G, RT, false>(a, tiles, s);
}

// Launch shape by input width (nblk = N/32 blocks).  Inputs that fit one
// K-chunk use the persistent kernel; wider ones the tile-per-workgroup one.
hipError_t launch_gemv(const GemvSeg* segs, int nseg, uint32_t nblk, const uint4* xd, hipStream_t s,
                       const GemvDecode* dec) {
    if (nseg < 1 || nseg > 4) return hipErrorInvalidValue;
    if (nblk <= 64) return run_gemv_p<1, 1, 4, 4>(segs, nseg, nblk, xd, nullptr, s, dec);
    if (nblk <= 128) return run_gemv_p<1, 2, 4, 2>(segs, nseg, nblk, xd, nullptr, s, dec);
    if (nblk <= 256) return run_gemv_p<2, 2, 1, 4>(segs, nseg, nblk, xd, nullptr, s, dec);
    if (nblk <= 448) return run_gemv_p<7, 1, 1, 8>(segs, nseg, nblk, xd, nullptr, s, dec);
    if (nblk <= 512) return run_gemv_p<8, 1, 1, 8>(segs, nseg, nblk, xd, nullptr, s, dec);
    return run_gemv<8, 2, 1, 16, 4>(segs, nseg, nblk, xd, s, dec);
}

// h = silu(W_gate . n) * (W_up . n), n = RMSNorm(x) with weight norm_w (the
// norm made in the prologue, the factor applied to both products), from the
// fp32 x[N], N <= 4096 (nblk <= 128).
hipError_t launch_gemv_swiglu(const uint8_t* w_gate, const uint8_t* w_up, uint32_t M, uint32_t N, const float* x,
                              const float* norm_w, float eps, float* h, hipStream_t s) {
    if (N == 0 || N % 32 != 0 || N / 32 > 128 || !w_gate || !w_up || !x || !norm_w || !h) return hipErrorInvalidValue;
    GemvArgs a{};
    a.w[0] = w_gate;
    a.w[1] = w_up;
    a.y[0] = h;
    a.M[0] = M;
    constexpr int kRT = 2;  // one gate and one up row per tile: one element of h
    const uint32_t tiles = (M + kRT / 2 - 1) / (kRT / 2);
    a.tile_end[0] = a.tile_end[1] = a.tile_end[2] = a.tile_end[3] = tiles;
    a.nseg = 1;
    a.nblk = N / 32;
    a.pad = xd_pad(a.nblk);
    a.xf = x;
    a.xnorm_w = norm_w;
    a.eps = eps;
    if (tiles == 0) return hipSuccess;
    return launch_gemv_p<1, 2, 4, kRT, true, true>(a, tiles, s);
}

// fp32 input: inputs of up to kGemvF32MaxBlk blocks are converted inside the
// GEMV (one launch); wider ones go through k_xprep into ws first.
hipError_t launch_gemv_f32(const GemvSeg* segs, int nseg, uint32_t N, const float* x, uint4* ws, hipStream_t s,
                           const GemvDecode* dec) {
    if (nseg < 1 || nseg > 4 || N == 0 || N % 32 != 0) return hipErrorInvalidValue;
    if (dec && dec->in_part) return hipErrorInvalidValue;
    const uint32_t nblk = N / 32;
    if (nblk <= 64) return run_gemv_p<1, 1, 4, 4>(segs, nseg, nblk, nullptr, x, s, dec);
    if (nblk <= 128) return run_gemv_p<1, 2, 4, 2>(segs, nseg, nblk, nullptr, x, s, dec);
    if (nblk <= 256) return run_gemv_p<2, 2, 1, 4>(segs, nseg, nblk, nullptr, x, s, dec);
    if (nblk <= 448) return run_gemv_p<7, 1, 1, 8>(segs, nseg, nblk, nullptr, x, s, dec);
    if (nblk <= 512) return run_gemv_p<8, 1, 1, 8>(segs, nseg, nblk, nullptr, x, s, dec);
    if (!ws || (dec && dec->norm_w)) return hipErrorInvalidValue;
    hipError_t e = launch_xprep(x, N, nullptr, 0.0f, nullptr, ws, s);
    if (e != hipSuccess) return e;
    return run_gemv<8, 2, 1, 16, 4>(segs, nseg, nblk, ws, s, dec);
}

// LM-head form of launch_gemv_f32 (one segment, plain store, 2048 < N <=
// 4096): y = W . x with the optional RMSNorm of x (dec->norm_w), and the
// greedy argmax's partials of y written to amax (values [0, n), first
// indices [n, 2n) as uint32), n = *n_part <= cap.  hipErrorNotSupported for
// other shapes (the caller then takes the separate argmax pass).
hipError_t launch_gemv_f32_amax(const GemvSeg& seg, uint32_t N, const float* x, const GemvDecode* dec, float* amax,
                                uint32_t cap, uint32_t* n_part, hipStream_t s) {
    if (!x || !amax || !n_part || !seg.w || !seg.y || seg.M == 0) return hipErrorInvalidValue;
    if (seg.res || seg.hd || seg.rope || (dec && (dec->pos || dec->in_part))) return hipErrorNotSupported;
    if (N % 32 != 0 || N / 32 <= 64 || N / 32 > 128) return hipErrorNotSupported;
    constexpr int kRT = 2;
    GemvArgs a{};
    a.w[0] = seg.w;
    a.y[0] = seg.y;
    a.M[0] = seg.M;
    const uint32_t tiles = (seg.M + kRT - 1) / kRT;
    a.tile_end[0] = a.tile_end[1] = a.tile_end[2] = a.tile_end[3] = tiles;
    a.nseg = 1;
    a.nblk = N / 32;
    a.pad = xd_pad(a.nblk);
    a.xf = x;
    a.xnorm_w = dec ? dec->norm_w : nullptr;
    a.eps = dec ? dec->eps : 0.0f;
    a.amax = amax;
    const uint32_t grid = gemv_p_grid<1, 2, 4, kRT, true, false, true>(tiles);
    if (grid > cap) return hipErrorNotSupported;
    *n_part = grid;
    return launch_gemv_p<1, 2, 4, kRT, true, false, true>(a, tiles, s);
}

}  // namespace qh
