// qh_digits.hpp -- device code that turns fp32 activations into the signed
// 4-bit digit planes consumed by the Q4_0 GEMV (k_q4.hip).  Any kernel that
// produces a GEMV input can emit its digits directly with prep_lane().
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

namespace qh {

// Per 32-element block of x:
//  * level 1: k with |A_e| <= kDigitMax for A_e = round(x_e * 2^k) (23-24
//    significant bits for the block maximum), stored as 6 balanced base-16
//    digit planes of 8 signed nibbles per dword (plane p, dword i holds
//    elements 8i..8i+7);
//  * a meta word (k, z, wide, 0): z = 0, or NaN when the block holds a NaN
//    or infinity (every dot product with the block is then NaN);
//  * level 2, for "wide" blocks only: the residual B_e = round((x_e * 2^k -
//    A_e) * 2^23) in 6 more planes.  A + 2^-23 B holds every element within
//    2^21 of the block maximum exactly (x * 2^k >= 1 there: the block
//    maximum lands at 2^21.9 or above; just below, an element can keep 24
//    bits instead).  The planes of a block that is not
//    wide are left unwritten; consumers read level 2 only through the flag.
// A block is wide unless, whichever 6 of its elements are removed, the rest
// keep a magnitude sum of at least 3/64 of the block maximum (level-1
// units).  Otherwise a few activation outliers set the step, and where they
// meet zero weights the remaining elements keep only the bits below the
// outliers' own.  The test takes lower bounds of that remainder that need
// no sort: for any threshold t, (sum of all but the 6 largest |A_e|) >=
// sum_e min(|A_e|, t) - 6 t, here at t = max|A| (the plain magnitude sum,
// which settles ordinary blocks; the clamped sums are then skipped), then
// max|A| / 16 and max|A| / 64 (the block is wide when all three bounds
// fall below 3/64 of max|A|).  So a block holding up to 6 outliers is wide
// whenever its other elements sum to less than 3/64 of them: 1..6 outliers
// of 1e3 or more among N(0,1) values always are.  N(0,1) inputs never
// flag; heavy-tailed ones rarely (SwiGLU products of N(0, 8^2) gates and
// ups: 3e-4 of their blocks; Student t3: 8e-6).  The sums are of exact
// integers, so every producer below sets the same flag.
// Layout: uint4 xd[13][pad]: planes 0..5, the meta word, planes 7..12.
//
// prep_lane: 32 consecutive lanes own one block (lane = element); block max,
// NaN/Inf flag and the clamped level-1 magnitude sums by cross-lane reductions, then
// the digits and the 8-lane OR that packs each plane dword.  Lanes 0..5 of
// each 8-lane group store the dwords of plane q (and of plane 7 + q for a
// wide block), lanes 6..7 of the first two groups store the meta word.
// Every lane of the wave must call it (it uses cross-lane operations).
constexpr int kDigitMax = 7829367;         // 7 * (16^6 - 1) / 15: largest 6-digit balanced value
constexpr uint32_t kDigitBias = 8947848u;  // 8 * (16^6 - 1) / 15
constexpr uint32_t kXdMeta = 6;            // plane index of (k, z, wide, 0)
constexpr uint32_t kXdLo = 7;              // first level-2 plane
constexpr float kLoInv = 1.1920928955078125e-07f;  // 2^-23, the weight of level 2
// A block's integer dot with level-1 (or level-2) digits: 32 products of a
// weight digit (|q - 8| <= 8) and an integer of at most kDigitMax.
static_assert(32LL * 8 * kDigitMax < (1LL << 31), "a block's integer dot fits int32");
static_assert(kDigitMax == 7 * ((1 << 24) - 1) / 15 && kDigitBias == 8u * ((1u << 24) - 1u) / 15u,
              "6 balanced base-16 digits");

// The wide test, in two stages.  maybe_wide: the bound from the magnitude
// sum asum = sum_e |A_e| falls below 3 (amax >> 6); block_wide: so do the
// bounds from c1 = sum_e min(|A_e|, amax >> 4) and c2 = sum_e min(|A_e|,
// amax >> 6) (needed only when maybe_wide holds).
__host__ __device__ __forceinline__ bool maybe_wide(int amax, int asum) { return asum - 6 * amax < 3 * (amax >> 6); }
__host__ __device__ __forceinline__ bool block_wide(int amax, int c1, int c2) {
    const int t1 = amax >> 4, t2 = amax >> 6;
    return c1 - 6 * t1 < 3 * t2 && c2 - 6 * t2 < 3 * t2;
}

// Cross-lane steps on the DPP datapath (full-rate VALU, no LDS round trip):
// quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2), and
// within a row of 16 the half mirror (lane i <-> 7 - i of each 8) and the
// mirror (lane i <-> 15 - i).  Applied in that order with an associative,
// commutative op they reduce groups of 4, 8 and 16 lanes into every lane.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t quad_max_u(uint32_t v) {
    v = __builtin_elementwise_max(v, dpp_u<0xB1>(v));
    return __builtin_elementwise_max(v, dpp_u<0x4E>(v));
}
__device__ __forceinline__ int quad_sum_i(int v) {
    v += (int)dpp_u<0xB1>((uint32_t)v);
    return v + (int)dpp_u<0x4E>((uint32_t)v);
}
// Over the 32 lanes of a half wave: 16-lane rows by DPP, then one swap of
// the row pair.
__device__ __forceinline__ float half_max_f(float v) {
    uint32_t b = __float_as_uint(v);
    v = fmaxf(v, __uint_as_float(dpp_u<0xB1>(b)));
    v = fmaxf(v, __uint_as_float(dpp_u<0x4E>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_u<0x141>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_u<0x140>(__float_as_uint(v))));
    return fmaxf(v, __shfl_xor(v, 16, 32));
}
__device__ __forceinline__ int half_sum_i(int v) {
    v = quad_sum_i(v);
    v += (int)dpp_u<0x141>((uint32_t)v);
    v += (int)dpp_u<0x140>((uint32_t)v);
    return v + __shfl_xor(v, 16, 32);
}

// Level-2 integer of one element given t = x * 2^k and a = round(t):
// t - a is exact in fp32, and so is its scaling by 2^23.
__device__ __forceinline__ int lo_int(float t, float a) { return (int)rintf((t - a) * 8388608.0f); }

__device__ inline void prep_lane(float v, uint32_t c, bool store, uint32_t pad, uint32_t* __restrict__ xd) {
    const int e = threadIdx.x & 31;
    const float a = fabsf(v);
    const bool bad_here = !(a <= FLT_MAX);  // NaN or infinity
    const float m = half_max_f(bad_here ? 0.0f : a);
    const uint64_t bm = __ballot(bad_here);
    const uint32_t grp = (threadIdx.x & 32) ? (uint32_t)(bm >> 32) : (uint32_t)bm;
    const bool bad = grp != 0u;
    int k = 0;
    if (!bad && m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m);  // m < 2^E
        k = 23 - E;
        if (rintf(ldexpf(m, k)) > (float)kDigitMax) k -= 1;
    }
    const float t = bad ? 0.0f : ldexpf(v, k);
    const float ar = rintf(t);
    const int xi = (int)ar;
    const int amax = bad ? 0 : (int)rintf(ldexpf(m, k));
    const int ax = xi < 0 ? -xi : xi;
    const bool maybe = !bad && maybe_wide(amax, half_sum_i(ax));
    bool wide = false;
    if (__ballot(maybe) != 0ull) {  // wave-uniform: every lane takes part in the sums
        const int c1 = half_sum_i(min(ax, amax >> 4));
        const int c2 = half_sum_i(min(ax, amax >> 6));
        wide = maybe && block_wide(amax, c1, c2);
    }
    const int sh = 4 * (e & 7);
    const int q = e & 7, i = e >> 3;
    // Packs one 6-digit value per lane into plane dwords (8-lane OR) and
    // returns the dword of plane q (lanes with q < 6).
    auto pack = [&](uint32_t u) {
        uint32_t pl[6];
#pragma unroll
        for (int p = 0; p < 6; ++p) pl[p] = ((u >> (4 * p)) & 15u) << sh;
#pragma unroll
        for (int off = 1; off < 8; off <<= 1)
#pragma unroll
            for (int p = 0; p < 6; ++p) pl[p] |= __shfl_xor(pl[p], off, 8);
        uint32_t val = pl[0];
#pragma unroll
        for (int p = 1; p < 6; ++p) val = (q == p) ? pl[p] : val;
        return val ^ 0x88888888u;
    };
    const uint32_t val = pack((uint32_t)(xi + (int)kDigitBias));  // 6 unsigned nibbles = digit + 8
    uint32_t val2 = 0u;
    if (__ballot(wide) != 0ull) val2 = pack((uint32_t)((wide ? lo_int(t, ar) : 0) + (int)kDigitBias));
    if (!store) return;
    if (q < 6) {
        xd[((size_t)q * pad + c) * 4 + i] = val;
        if (wide) xd[((size_t)(kXdLo + q) * pad + c) * 4 + i] = val2;
    } else if (i < 2) {
        const float z = bad ? __builtin_nanf("") : 0.0f;
        const uint32_t w = (uint32_t)(2 * i + (q - 6));  // meta dword
        const uint32_t val = w == 0 ? (uint32_t)k : (w == 1 ? __float_as_uint(z) : (w == 2 ? (uint32_t)wide : 0u));
        xd[((size_t)kXdMeta * pad + c) * 4 + w] = val;
    }
}

// Nibble transpose of 8 elements' biased 6-digit values u[0..8) (element
// 8i + e in u[e]): pl[p] gets digit p of element e in nibble e, XORed with
// 0x88888888 (signed digits).  It works on element pairs (u0, u1): lo =
// nibbles 0, 2, 4 of u0 in the low and of u1 in the high half of bytes 0..2,
// hi = nibbles 1, 3, 5 likewise; byte b of the four pairs' words is plane 2b
// (lo) or 2b+1 (hi), gathered with byte permutes.
__device__ __forceinline__ void planes8(const uint32_t (&u)[8], uint32_t (&pl)[6]) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
        const uint32_t u0 = u[2 * pr], u1 = u[2 * pr + 1];
        lo[pr] = (u0 & 0x0F0F0F0Fu) | ((u1 << 4) & 0xF0F0F0F0u);
        hi[pr] = ((u0 >> 4) & 0x0F0F0F0Fu) | (u1 & 0xF0F0F0F0u);
    }
    // t = (w0.b0, w1.b0, w0.b1, w1.b1), s = (w0.b2, w1.b2, -, -)
    const uint32_t tl01 = __builtin_amdgcn_perm(lo[1], lo[0], 0x05010400u);
    const uint32_t tl23 = __builtin_amdgcn_perm(lo[3], lo[2], 0x05010400u);
    const uint32_t sl01 = __builtin_amdgcn_perm(lo[1], lo[0], 0x00000602u);
    const uint32_t sl23 = __builtin_amdgcn_perm(lo[3], lo[2], 0x00000602u);
    const uint32_t th01 = __builtin_amdgcn_perm(hi[1], hi[0], 0x05010400u);
    const uint32_t th23 = __builtin_amdgcn_perm(hi[3], hi[2], 0x05010400u);
    const uint32_t sh01 = __builtin_amdgcn_perm(hi[1], hi[0], 0x00000602u);
    const uint32_t sh23 = __builtin_amdgcn_perm(hi[3], hi[2], 0x00000602u);
    pl[0] = __builtin_amdgcn_perm(tl23, tl01, 0x05040100u) ^ 0x88888888u;
    pl[2] = __builtin_amdgcn_perm(tl23, tl01, 0x07060302u) ^ 0x88888888u;
    pl[4] = __builtin_amdgcn_perm(sl23, sl01, 0x05040100u) ^ 0x88888888u;
    pl[1] = __builtin_amdgcn_perm(th23, th01, 0x05040100u) ^ 0x88888888u;
    pl[3] = __builtin_amdgcn_perm(th23, th01, 0x07060302u) ^ 0x88888888u;
    pl[5] = __builtin_amdgcn_perm(sh23, sh01, 0x05040100u) ^ 0x88888888u;
}

// Block exponent k from the unsigned maximum of the bit patterns shifted left
// by one (the sign dropped), which also flags infinities and NaNs (pattern
// >= 0xFF000000).
__device__ __forceinline__ int block_k(uint32_t mb, bool bad, float& m) {
    m = __uint_as_float(mb >> 1);
    int k = 0;
    if (!bad && m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m);  // m < 2^E
        k = 23 - E;
        if (rintf(ldexpf(m, k)) > (float)kDigitMax) k -= 1;
    }
    return k;
}

// One thread converts one whole 32-element block v[0..32) into the digit
// planes prep_lane produces for it: out[0..5] = planes 0..5 (dword i holds
// elements 8i..8i+7, already XORed with 0x88888888), out[6] = the meta word
// (k, z, wide, 0), out[7..12] = level 2 (zero unless wide).  A NaN/Inf
// block gets z = NaN and the digits of the zero block.
__device__ __forceinline__ void prep_block(const float (&v)[32], uint4 (&out)[13]) {
    uint32_t mb = 0u;
#pragma unroll
    for (int e = 0; e < 32; ++e) mb = __builtin_elementwise_max(mb, __float_as_uint(v[e]) << 1);
    const bool bad = mb >= 0xFF000000u;
    float m;
    const int k = block_k(mb, bad, m);
    const int amax = bad ? 0 : (int)rintf(ldexpf(m, k));
    uint32_t pl[6][4];
    int asum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t u[8], p8[6];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int a = bad ? 0 : (int)rintf(ldexpf(v[8 * i + e], k));
            asum += a < 0 ? -a : a;
            u[e] = (uint32_t)(a + (int)kDigitBias);
        }
        planes8(u, p8);
#pragma unroll
        for (int p = 0; p < 6; ++p) pl[p][i] = p8[p];
    }
    bool wide = false;
    if (!bad && maybe_wide(amax, asum)) {
        const int t1 = amax >> 4, t2 = amax >> 6;
        int c1 = 0, c2 = 0;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const int a = (int)rintf(ldexpf(v[e], k));
            const int ax = a < 0 ? -a : a;
            c1 += min(ax, t1);
            c2 += min(ax, t2);
        }
        wide = block_wide(amax, c1, c2);
    }
#pragma unroll
    for (int p = 0; p < 6; ++p) out[p] = make_uint4(pl[p][0], pl[p][1], pl[p][2], pl[p][3]);
    out[kXdMeta] = make_uint4((uint32_t)k, __float_as_uint(bad ? __builtin_nanf("") : 0.0f), (uint32_t)wide, 0u);
#pragma unroll
    for (int p = 0; p < 6; ++p) out[kXdLo + p] = make_uint4(0u, 0u, 0u, 0u);
    if (wide) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t u[8], p8[6];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float t = ldexpf(v[8 * i + e], k);
                u[e] = (uint32_t)(lo_int(t, rintf(t)) + (int)kDigitBias);
            }
            planes8(u, p8);
#pragma unroll
            for (int p = 0; p < 6; ++p) {
                uint4& o = out[kXdLo + p];
                if (i == 0) o.x = p8[p];
                if (i == 1) o.y = p8[p];
                if (i == 2) o.z = p8[p];
                if (i == 3) o.w = p8[p];
            }
        }
    }
}

// prep_block split over the 4 lanes of an aligned lane quad: lane i of the
// quad holds elements 8i..8i+7 of the block in v and gets dword i of every
// level-1 plane (pl, already XORed with 0x88888888), the block's k and z
// words, its level-1 maximum amax and maybe = maybe_wide (the cheap first
// stage of the wide test).  The block maximum and magnitude sum are combined
// across the quad, so all 4 lanes must call it together; the digits are
// those of prep_block bit for bit.  quarter_wide completes the wide test
// (the flag of prep_block), and prep_quarter_lo gives the same lane's dwords
// of the level-2 planes of a wide block.  The second stage is kept apart so
// a caller converting several blocks per lane runs it once, after all of
// them, and only when some lane of the wave needs it.
__device__ __forceinline__ void prep_quarter(const float (&v)[8], uint32_t (&pl)[6], uint32_t& k_out,
                                             uint32_t& z_out, int& amax_out, bool& maybe_out) {
    uint32_t mb = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) mb = __builtin_elementwise_max(mb, __float_as_uint(v[e]) << 1);
    mb = quad_max_u(mb);
    const bool bad = mb >= 0xFF000000u;
    float m;
    const int k = block_k(mb, bad, m);
    const int amax = bad ? 0 : (int)rintf(ldexpf(m, k));
    uint32_t u[8];
    int asum = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int a = bad ? 0 : (int)rintf(ldexpf(v[e], k));
        asum += a < 0 ? -a : a;
        u[e] = (uint32_t)(a + (int)kDigitBias);
    }
    planes8(u, pl);
    asum = quad_sum_i(asum);
    k_out = (uint32_t)k;
    z_out = __float_as_uint(bad ? __builtin_nanf("") : 0.0f);
    amax_out = amax;
    maybe_out = !bad && maybe_wide(amax, asum);
}

// Second stage of the wide test for a block prep_quarter converted (k,
// amax, maybe from it); all 4 lanes of the quad call it together.
__device__ __forceinline__ bool quarter_wide(const float (&v)[8], int k, int amax, bool maybe) {
    const int t1 = amax >> 4, t2 = amax >> 6;
    int c1 = 0, c2 = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int a = maybe ? (int)rintf(ldexpf(v[e], k)) : 0;
        const int ax = a < 0 ? -a : a;
        c1 += min(ax, t1);
        c2 += min(ax, t2);
    }
    c1 = quad_sum_i(c1);
    c2 = quad_sum_i(c2);
    return maybe && block_wide(amax, c1, c2);
}

__device__ __forceinline__ void prep_quarter_lo(const float (&v)[8], int k, uint32_t (&pl2)[6]) {
    uint32_t u2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float t = ldexpf(v[e], k);
        u2[e] = (uint32_t)(lo_int(t, rintf(t)) + (int)kDigitBias);
    }
    planes8(u2, pl2);
}

// Integer dots of R*J blocks (already loaded) against the level-1 digit
// planes: plane by plane across all blocks, each plane a 4-deep dot8 chain
// of its own, planes combined by P = (P << 4) + S_p, so the independent
// chains of different blocks interleave.  P is exact (|P| <= 32*8*kDigitMax
// < 2^31).
template <int R, int J>
__device__ __forceinline__ void dot_planes(const uint32_t (&wq)[R][J][4], const uint4 (&xp)[J][6], int (&P)[R][J]) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) P[r][j] = 0;
#pragma unroll
    for (int p = 5; p >= 0; --p)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < J; ++j) {
                int sp = __builtin_amdgcn_sdot8((int)wq[r][j][0], (int)xp[j][p].x, 0, false);
                sp = __builtin_amdgcn_sdot8((int)wq[r][j][1], (int)xp[j][p].y, sp, false);
                sp = __builtin_amdgcn_sdot8((int)wq[r][j][2], (int)xp[j][p].z, sp, false);
                sp = __builtin_amdgcn_sdot8((int)wq[r][j][3], (int)xp[j][p].w, sp, false);
                P[r][j] = (int)((uint32_t)P[r][j] << 4) + sp;
            }
}

template <int R, int J>
__device__ __forceinline__ void weight_digits(const uint4 (&q)[R][J], uint32_t (&wq)[R][J][4]) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            wq[r][j][0] = q[r][j].x ^ 0x88888888u;
            wq[r][j][1] = q[r][j].y ^ 0x88888888u;
            wq[r][j][2] = q[r][j].z ^ 0x88888888u;
            wq[r][j][3] = q[r][j].w ^ 0x88888888u;
        }
}

// Level 1 only: acc += ldexp(fma(s, (float)P, z), -k) per block.
template <int R, int J>
__device__ __forceinline__ void dot_batch(const uint4 (&q)[R][J], const float (&s)[R][J], const uint4 (&xp)[J][6],
                                          const int (&kk)[J], const float (&zz)[J], const bool (&ok)[J],
                                          float (&acc)[R]) {
    uint32_t wq[R][J][4];
    weight_digits<R, J>(q, wq);
    int P[R][J];
    dot_planes<R, J>(wq, xp, P);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float sc = ok[j] ? s[r][j] : 0.0f;
            const float c = fmaf(sc, (float)P[r][j], zz[j]);
            acc[r] += ldexpf(c, -kk[j]);
        }
}

// Both levels: each block adds ldexp(fma(s, fma((float)Q, 2^-23,
// (float)P), z), -k), the level-2 planes read by lo(j, p, salt) one plane at
// a time for the columns whose wide flag wd[j] is set (Q = 0 for the
// others, which then get exactly dot_batch's value).  The level-2 planes do not change from one call to the
// next: lo adds the opaque zero `salt` to its column address, so the
// compiler can neither hoist the loads out of the caller's tile loop (where
// they would hold 24*J registers for the whole kernel) nor issue all planes
// at once; the slow path trades load latency for registers, and the
// kernel's occupancy stays that of level 1.
template <int R, int J, typename Lo>
__device__ __forceinline__ void dot_batch2(const uint4 (&q)[R][J], const float (&s)[R][J], const uint4 (&xp)[J][6],
                                           Lo lo, const int (&kk)[J], const float (&zz)[J], const bool (&ok)[J],
                                           const uint32_t (&wd)[J], float (&acc)[R]) {
    uint32_t wq[R][J][4];
    weight_digits<R, J>(q, wq);
    int P[R][J], Q[R][J];
    dot_planes<R, J>(wq, xp, P);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) Q[r][j] = 0;
    uint32_t salt = 0;
    asm volatile("" : "+v"(salt));
#pragma unroll
    for (int p = 5; p >= 0; --p) {
        uint4 x2[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            // Only a wide block's level-2 planes are written.
            const uint4 v = lo(j, p, salt);
            x2[j] = wd[j] ? v : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < J; ++j) {
                int sp = __builtin_amdgcn_sdot8((int)wq[r][j][0], (int)x2[j].x, 0, false);
                sp = __builtin_amdgcn_sdot8((int)wq[r][j][1], (int)x2[j].y, sp, false);
                sp = __builtin_amdgcn_sdot8((int)wq[r][j][2], (int)x2[j].z, sp, false);
                sp = __builtin_amdgcn_sdot8((int)wq[r][j][3], (int)x2[j].w, sp, false);
                Q[r][j] = (int)((uint32_t)Q[r][j] << 4) + sp;
            }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float sc = ok[j] ? s[r][j] : 0.0f;
            const float t = fmaf((float)Q[r][j], kLoInv, (float)P[r][j]);
            const float c = fmaf(sc, t, zz[j]);
            acc[r] += ldexpf(c, -kk[j]);
        }
}

// Loads a lane's level-1 digit planes and meta word for J block columns:
// column j is cols[j] when ok[j], else it reads zeros.  Buffer loads with an
// offset past the resource's size return zero, so the loads stay
// unconditional (no branch, no extra wait) whatever the column mask.
template <int J>
__device__ __forceinline__ void load_digits(const uint4* xd, uint32_t pad, const uint32_t (&cols)[J],
                                            const bool (&ok)[J], uint4 (&xp)[J][6], int (&kk)[J],
                                            float (&zz)[J], uint32_t (&wd)[J]) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)xd, 0, (int)(13u * pad * 16u), 0x00020000);
    const uint32_t kOut = 0x7FFFFFF0u;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int p = 0; p < 6; ++p) {
            const v4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, ok[j] ? ((uint32_t)p * pad + cols[j]) * 16u : kOut, 0, 0);
            xp[j][p] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        const v4 m = __builtin_amdgcn_raw_buffer_load_b128(rs, ok[j] ? (kXdMeta * pad + cols[j]) * 16u : kOut, 0, 0);
        kk[j] = (int)m[0];
        zz[j] = __uint_as_float(m[1]);
        wd[j] = m[2];
    }
}

// Level-2 plane p of column col (zero when !ok), from HBM; salt is added to
// the per-lane offset (see dot_batch2).
__device__ __forceinline__ uint4 load_lo_plane(const uint4* xd, uint32_t pad, uint32_t col, bool ok, int p,
                                               uint32_t salt) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)xd, 0, (int)(13u * pad * 16u), 0x00020000);
    const v4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (ok ? col * 16u : 0x7FFFFFF0u) + salt,
                                                       (int)((kXdLo + (uint32_t)p) * pad * 16u), 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

}  // namespace qh
