// qh_digits.hpp -- device code that turns fp32 activations into the signed
// 4-bit digit planes consumed by the Q4_0 GEMV (k_q4.hip).  Any kernel that
// produces a GEMV input can emit its digits directly with prep_lane().
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

namespace qh {

// Per 32-element block of x: k with |round(x * 2^k)| <= kDigitMax (23-24
// significant bits for the block maximum), the 6 balanced base-16 digits of
// x_int = round(x * 2^k) stored as 6 planes of 8 signed nibbles per dword
// (plane p, dword i holds elements 8i..8i+7), and a word z = 0 (or NaN when
// the block holds a NaN or infinity, which makes every dot product with the
// block NaN).  Layout: uint4 xd[7][pad]; planes 0..5, then (k, z, 0, 0).
//
// prep_lane: 32 consecutive lanes own one block (lane = element); block max
// and NaN/Inf flag by cross-lane reductions, then the digits and the 8-lane
// OR that packs each plane dword.  Lanes 0..5 of each 8-lane group store
// plane dwords, lanes 6..7 of the first group store (k, z).  Every lane of
// the wave must call it (it uses cross-lane operations).
constexpr int kDigitMax = 7829367;         // 7 * (16^6 - 1) / 15: largest 6-digit balanced value
constexpr uint32_t kDigitBias = 8947848u;  // 8 * (16^6 - 1) / 15

__device__ inline void prep_lane(float v, uint32_t c, bool store, uint32_t pad, uint32_t* __restrict__ xd) {
    const int e = threadIdx.x & 31;
    const float a = fabsf(v);
    const bool bad_here = !(a <= FLT_MAX);  // NaN or infinity
    float m = bad_here ? 0.0f : a;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 32));
    const uint64_t bm = __ballot(bad_here);
    const uint32_t grp = (threadIdx.x & 32) ? (uint32_t)(bm >> 32) : (uint32_t)bm;
    const bool bad = grp != 0u;
    int k = 0;
    if (!bad && m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m);  // m < 2^E
        k = 23 - E;
        if (rintf(ldexpf(m, k)) > (float)kDigitMax) k -= 1;
    }
    const int xi = bad ? 0 : (int)rintf(ldexpf(v, k));
    const uint32_t u = (uint32_t)(xi + (int)kDigitBias);  // 6 unsigned nibbles = digit + 8
    const int sh = 4 * (e & 7);
    uint32_t pl[6];
#pragma unroll
    for (int p = 0; p < 6; ++p) pl[p] = ((u >> (4 * p)) & 15u) << sh;
#pragma unroll
    for (int off = 1; off < 8; off <<= 1)
#pragma unroll
        for (int p = 0; p < 6; ++p) pl[p] |= __shfl_xor(pl[p], off, 8);
    if (!store) return;
    const int q = e & 7, i = e >> 3;
    if (q < 6) {
        uint32_t val = pl[0];
#pragma unroll
        for (int p = 1; p < 6; ++p) val = (q == p) ? pl[p] : val;
        xd[((size_t)q * pad + c) * 4 + i] = val ^ 0x88888888u;
    } else if (i == 0) {
        const float z = bad ? __builtin_nanf("") : 0.0f;
        xd[((size_t)6 * pad + c) * 4 + (q - 6)] = (q == 6) ? (uint32_t)k : __float_as_uint(z);
    }
}

// One thread converts one whole 32-element block v[0..32) into the digit
// planes prep_lane produces for it: out[0..5] = planes 0..5 (dword i holds
// elements 8i..8i+7, already XORed with 0x88888888), out[6] = (k, z, 0, 0).
// The block maximum is an unsigned maximum over the bit patterns shifted
// left by one (the sign dropped), which also flags infinities and NaNs
// (pattern >= 0xFF000000).  Such a block gets z = NaN; its digits are then
// those of the zero block.  The nibble transpose works on element pairs
// (u0, u1): lo = nibbles 0, 2, 4 of u0 in the low and of u1 in the high
// half of bytes 0..2, hi = nibbles 1, 3, 5 likewise; byte b of the four
// pairs' words of 8 elements is plane 2b (lo) or 2b+1 (hi), gathered with
// byte permutes.
__device__ __forceinline__ void prep_block(const float (&v)[32], uint4 (&out)[7]) {
    uint32_t mb = 0u;
#pragma unroll
    for (int e = 0; e < 32; ++e) mb = __builtin_elementwise_max(mb, __float_as_uint(v[e]) << 1);
    const bool bad = mb >= 0xFF000000u;
    const float m = __uint_as_float(mb >> 1);
    int k = 0;
    if (!bad && m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m);  // m < 2^E
        k = 23 - E;
        if (rintf(ldexpf(m, k)) > (float)kDigitMax) k -= 1;
    }
    uint32_t pl[6][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
            const float a0 = bad ? 0.0f : v[8 * i + 2 * pr], a1 = bad ? 0.0f : v[8 * i + 2 * pr + 1];
            const uint32_t u0 = (uint32_t)((int)rintf(ldexpf(a0, k)) + (int)kDigitBias);
            const uint32_t u1 = (uint32_t)((int)rintf(ldexpf(a1, k)) + (int)kDigitBias);
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
        pl[0][i] = __builtin_amdgcn_perm(tl23, tl01, 0x05040100u);
        pl[2][i] = __builtin_amdgcn_perm(tl23, tl01, 0x07060302u);
        pl[4][i] = __builtin_amdgcn_perm(sl23, sl01, 0x05040100u);
        pl[1][i] = __builtin_amdgcn_perm(th23, th01, 0x05040100u);
        pl[3][i] = __builtin_amdgcn_perm(th23, th01, 0x07060302u);
        pl[5][i] = __builtin_amdgcn_perm(sh23, sh01, 0x05040100u);
    }
#pragma unroll
    for (int p = 0; p < 6; ++p)
        out[p] = make_uint4(pl[p][0] ^ 0x88888888u, pl[p][1] ^ 0x88888888u, pl[p][2] ^ 0x88888888u,
                            pl[p][3] ^ 0x88888888u);
    out[6] = make_uint4((uint32_t)k, __float_as_uint(bad ? __builtin_nanf("") : 0.0f), 0u, 0u);
}

// prep_block split over the 4 lanes of an aligned lane quad: lane i of the
// quad holds elements 8i..8i+7 of the block in v and gets dword i of every
// plane (pl[p], already XORed with 0x88888888) and the block's (k, z) word
// pair.  The block maximum is combined across the quad, so all 4 lanes must
// call it together; the digits are those of prep_block bit for bit.
__device__ __forceinline__ void prep_quarter(const float (&v)[8], uint32_t (&pl)[6], uint32_t& k_out,
                                             uint32_t& z_out) {
    uint32_t mb = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) mb = __builtin_elementwise_max(mb, __float_as_uint(v[e]) << 1);
    mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, 1));
    mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, 2));
    const bool bad = mb >= 0xFF000000u;
    const float m = __uint_as_float(mb >> 1);
    int k = 0;
    if (!bad && m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m);  // m < 2^E
        k = 23 - E;
        if (rintf(ldexpf(m, k)) > (float)kDigitMax) k -= 1;
    }
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
        const float a0 = bad ? 0.0f : v[2 * pr], a1 = bad ? 0.0f : v[2 * pr + 1];
        const uint32_t u0 = (uint32_t)((int)rintf(ldexpf(a0, k)) + (int)kDigitBias);
        const uint32_t u1 = (uint32_t)((int)rintf(ldexpf(a1, k)) + (int)kDigitBias);
        lo[pr] = (u0 & 0x0F0F0F0Fu) | ((u1 << 4) & 0xF0F0F0F0u);
        hi[pr] = ((u0 >> 4) & 0x0F0F0F0Fu) | (u1 & 0xF0F0F0F0u);
    }
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
    k_out = (uint32_t)k;
    z_out = __float_as_uint(bad ? __builtin_nanf("") : 0.0f);
}

// Integer dots of R*J blocks (already loaded) against the x digit planes,
// accumulated into acc[0..R): plane by plane across all blocks, each plane a
// 4-deep dot8 chain of its own, planes combined by P = (P << 4) + S_p, so
// the independent chains of different blocks interleave; then
// acc += ldexp(fma(s, (float)P, z), -k) per block.
template <int R, int J>
__device__ __forceinline__ void dot_batch(const uint4 (&q)[R][J], const float (&s)[R][J], const uint4 (&xp)[J][6],
                                          const int (&kk)[J], const float (&zz)[J], const bool (&ok)[J],
                                          float (&acc)[R]) {
    int P[R][J];
    uint32_t wq[R][J][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            wq[r][j][0] = q[r][j].x ^ 0x88888888u;
            wq[r][j][1] = q[r][j].y ^ 0x88888888u;
            wq[r][j][2] = q[r][j].z ^ 0x88888888u;
            wq[r][j][3] = q[r][j].w ^ 0x88888888u;
            P[r][j] = 0;
        }
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
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float sc = ok[j] ? s[r][j] : 0.0f;
            const float c = fmaf(sc, (float)P[r][j], zz[j]);
            acc[r] += ldexpf(c, -kk[j]);
        }
}

// Loads a lane's digit planes and (k, z) for J block columns: column j is
// cols[j] when ok[j], else it reads zeros.  Buffer loads with an offset past
// the resource's size return zero, so the loads stay unconditional (no
// branch, no extra wait) whatever the column mask.
template <int J>
__device__ __forceinline__ void load_digits(const uint4* xd, uint32_t pad, const uint32_t (&cols)[J],
                                            const bool (&ok)[J], uint4 (&xp)[J][6], int (&kk)[J],
                                            float (&zz)[J]) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)xd, 0, (int)(7u * pad * 16u), 0x00020000);
    const uint32_t kOut = 0x7FFFFFF0u;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int p = 0; p < 6; ++p) {
            const v4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, ok[j] ? ((uint32_t)p * pad + cols[j]) * 16u : kOut, 0, 0);
            xp[j][p] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        const v4 m = __builtin_amdgcn_raw_buffer_load_b128(rs, ok[j] ? (6u * pad + cols[j]) * 16u : kOut, 0, 0);
        kk[j] = (int)m[0];
        zz[j] = __uint_as_float(m[1]);
    }
}

}  // namespace qh
