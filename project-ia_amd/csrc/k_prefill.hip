// k_prefill.hip -- batched-prefill kernels for gfx950 other than the GEMM:
// token embedding rows, RoPE of the Q|K rows with the KV-cache stores, and
// the causal attention of T queries over the cache on fp32 matrix cores.
//
// The prefill computes what T successive decode steps compute (reference
// src/models/model.c:1655-1850 run with seq_len = 1 per token): token t at
// position pos0 + t attends the cached keys 0 .. pos0 + t.  (The reference's
// own seq_len > 1 branch normalizes only the first row, model.c:1108 and
// 1624, and attends only within the batch, model.c:1340-1440; a prompt
// continued at pos0 > 0 then ignores its cached keys.  This build keeps the
// token-by-token result for every seq_len.)
#include <hip/hip_runtime.h>

#include <algorithm>

#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "qh_prefill.hpp"
#include "qh_vec.hpp"

namespace qh {

typedef float f4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr uint32_t kPHd = 128;  // head_dim the prefill kernels are written for

__global__ __launch_bounds__(256) void k_embed_rows(const float* __restrict__ embd, const uint32_t* __restrict__ tok,
                                                    uint32_t dim, float* __restrict__ X) {
    const uint32_t t = blockIdx.y;
    const float4* src = reinterpret_cast<const float4*>(embd + (size_t)tok[t] * dim);
    float4* dst = reinterpret_cast<float4*>(X + (size_t)t * dim);
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < dim / 4; i += gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_embed_rows(const float* embd, const uint32_t* tok, uint32_t T, uint32_t dim, float* X,
                             hipStream_t s) {
    if (T == 0 || dim == 0 || dim % 4 != 0) return hipErrorInvalidValue;
    const uint32_t gx = (dim / 4 + 255) / 256;
    hipLaunchKernelGGL(k_embed_rows, dim3(gx, T), dim3(256), 0, s, embd, tok, dim, X);
    return hipGetLastError();
}

// RoPE pair (x0, x1) -> (x0*c - x1*s, x1*c + x0*s), reference
// src/ops/avx2/rope.c:244-285 with the table of position pos0 + t.
__device__ __forceinline__ float2 rope_pair(float2 x, float c, float sn) {
    const float a0 = x.x * c, b0 = x.y * sn;
    const float a1 = x.y * c, b1 = x.x * sn;
    return make_float2(a0 - b0, a1 + b1);
}

// Reduced Q|K|V pair (x0, x1) at column c of token t from the GEMM's split-K
// partials: (sum_s part[s][t][c..c+1]) * pm.x, NaN where pm.y is set (the
// order of k_gemm_reduce and gemm_store).
__device__ __forceinline__ float2 part_pair(const float* part, uint32_t split, size_t plane, float2 pm, size_t at) {
    float2 v = *reinterpret_cast<const float2*>(part + at);
    uint32_t sp = 1;
    // 8 loads in flight at a time; the sum stays sequential in split order
    for (; sp + 8 <= split; sp += 8) {
        float2 w[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const float2*>(part + (sp + u) * plane + at);
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            v.x += w[u].x;
            v.y += w[u].y;
        }
    }
    for (; sp < split; ++sp) {
        const float2 w = *reinterpret_cast<const float2*>(part + sp * plane + at);
        v.x += w.x;
        v.y += w.y;
    }
    v.x = v.x * pm.x;
    v.y = v.y * pm.x;
    if (pm.y != 0.0f) v = make_float2(__builtin_nanf(""), __builtin_nanf(""));
    return v;
}

__global__ __launch_bounds__(256) void k_rope_kv_rows(float* __restrict__ Q, const float* __restrict__ K,
                                                      const float* __restrict__ V, const float* __restrict__ ct,
                                                      const float* __restrict__ st, uint32_t pos0,
                                                      uint32_t n_heads, uint32_t n_kv, uint32_t max_seq,
                                                      float* __restrict__ kv_layer, const float* __restrict__ part,
                                                      uint32_t split, const float2* __restrict__ pmeta, uint32_t T) {
    const uint32_t t = blockIdx.x, P = pos0 + t;
    const uint32_t qd = n_heads * kPHd, kvd = n_kv * kPHd;
    const float* c = ct + (size_t)P * kPHd;
    const float* sn = st + (size_t)P * kPHd;
    float* q = Q + (size_t)t * qd;
    // reduction mode: the Q|K|V GEMM's partial row t, [q | k | v] columns
    const uint32_t ld = qd + 2 * kvd;
    const size_t plane = (size_t)T * ld, prow = (size_t)t * ld;
    const float2 pm = part ? pmeta[t] : make_float2(1.0f, 0.0f);
    // pairs are split over gridDim.y workgroups per token (more than one for
    // short prompts, whose rows are few)
    const uint32_t p0 = threadIdx.x + 256u * blockIdx.y, pstep = 256u * gridDim.y;
    for (uint32_t p = p0; p < qd / 2; p += pstep) {
        const uint32_t i = 2 * p, e = i % kPHd;
        float2* qp = reinterpret_cast<float2*>(q + i);
        const float2 x = part ? part_pair(part, split, plane, pm, prow + i) : *qp;
        *qp = rope_pair(x, c[e], sn[e]);
    }
    const float* k = K + (size_t)t * kvd;
    const float* v = V + (size_t)t * kvd;
    for (uint32_t p = p0; p < kvd / 2; p += pstep) {
        const uint32_t i = 2 * p, h = i / kPHd, e = i % kPHd;
        float* dst = kv_layer + ((size_t)h * max_seq + P) * 2 * kPHd;
        const float2 kx = part ? part_pair(part, split, plane, pm, prow + qd + i)
                               : *reinterpret_cast<const float2*>(k + i);
        const float2 vx = part ? part_pair(part, split, plane, pm, prow + qd + kvd + i)
                               : *reinterpret_cast<const float2*>(v + i);
        *reinterpret_cast<float2*>(dst + e) = rope_pair(kx, c[e], sn[e]);
        *reinterpret_cast<float2*>(dst + kPHd + e) = vx;
    }
}

hipError_t launch_rope_kv_rows(float* Q, const float* K, const float* V, const float* cos_tab,
                               const float* sin_tab, uint32_t pos0, uint32_t T, uint32_t n_heads, uint32_t n_kv,
                               uint32_t max_seq, float* kv_layer, hipStream_t s, const float* part, uint32_t split,
                               const float2* pmeta) {
    if (T == 0 || n_kv == 0 || (uint64_t)pos0 + T > max_seq || (part && (split == 0 || !pmeta)))
        return hipErrorInvalidValue;
    const uint32_t per_token = std::max(1u, std::min(8u, 256u / T));  // workgroups per token row
    hipLaunchKernelGGL(k_rope_kv_rows, dim3(T, per_token), dim3(256), 0, s, Q, K, V, cos_tab, sin_tab, pos0, n_heads,
                       n_kv, max_seq, kv_layer, part, split, pmeta, T);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Keys as fp16 hi/lo rows for the attention's q.k on fp16 matrix cores.
// Row j of KV head h (keys 0 .. n_keys-1) is scaled by 2^e, e chosen per
// row so that max|k'| lies in [2^14, 2^15) (e = 0 for an all-zero or
// non-finite row), and split as hi = rn(k'), lo = rn(k' - hi) (the
// subtraction is exact in fp32): 22 significant bits of every element within
// 2^17 of the row maximum, steps of 2^-24 (of k') below that.  With each
// row goes a flag: the key's V row holds a NaN or an infinity (its P.V terms
// must then be formed even where e_j = 0, as 0 * v_j is NaN).  Layout: halfs
// [n_kv][max_seq][hi 0..127 | lo 0..127], then int32 2e + flag [n_kv][max_seq].
// One 32-lane half of a wave per row, one float4 of K and of V per lane.
// ---------------------------------------------------------------------------
size_t prefill_khl_bytes(uint32_t n_kv, uint32_t max_seq) {
    const size_t rows = (size_t)n_kv * max_seq;
    return ((rows * 2 * kPHd * 2 + 255) & ~(size_t)255) + rows * 4;
}

__host__ __device__ inline int* khl_meta(void* khl, uint32_t n_kv, uint32_t max_seq) {
    const size_t rows = (size_t)n_kv * max_seq;
    return reinterpret_cast<int*>(static_cast<uint8_t*>(khl) + ((rows * 2 * kPHd * 2 + 255) & ~(size_t)255));
}

// Exponent e with max|x * 2^e| in [2^14, 2^15) for a finite m = max|x| > 0,
// else 0.
__device__ __forceinline__ int split_exp(float m) {
    return (m > 0.0f && m <= FLT_MAX) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
}

__global__ __launch_bounds__(256) void k_prefill_khl(const float* __restrict__ kv, uint32_t n_keys, uint32_t max_seq,
                                                     _Float16* __restrict__ khl, int* __restrict__ meta) {
    const uint32_t kvh = blockIdx.y;
    const uint32_t j = blockIdx.x * 8u + (threadIdx.x >> 5), c = threadIdx.x & 31u;
    if (j >= n_keys) return;  // uniform over the row's 32 lanes
    const size_t row = (size_t)kvh * max_seq + j;
    const float4 x = *reinterpret_cast<const float4*>(kv + row * (2 * kPHd) + 4 * c);
    const float4 vx = *reinterpret_cast<const float4*>(kv + row * (2 * kPHd) + kPHd + 4 * c);
    const bool vbad = !(fabsf(vx.x) <= FLT_MAX && fabsf(vx.y) <= FLT_MAX && fabsf(vx.z) <= FLT_MAX &&
                        fabsf(vx.w) <= FLT_MAX);
    const uint64_t vb = __ballot(vbad);
    const bool row_vbad = ((threadIdx.x & 32) ? (uint32_t)(vb >> 32) : (uint32_t)vb) != 0u;
    float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    if (!(x.x == x.x && x.y == x.y && x.z == x.z && x.w == x.w)) m = INFINITY;  // NaN: no scaling
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 32));
    const int e = split_exp(m);
    const float v[4] = {ldexpf(x.x, e), ldexpf(x.y, e), ldexpf(x.z, e), ldexpf(x.w, e)};
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hi[i] = (_Float16)v[i];
        lo[i] = (_Float16)(v[i] - (float)hi[i]);
    }
    _Float16* dst = khl + row * (2 * kPHd) + 4 * c;
    *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(hi);
    *reinterpret_cast<uint2*>(dst + kPHd) = *reinterpret_cast<const uint2*>(lo);
    if (c == 0) meta[row] = 2 * e + (row_vbad ? 1 : 0);
}

// ---------------------------------------------------------------------------
// Causal prefill attention: q.k on fp16 matrix cores (v_mfma_f32_16x16x32_f16
// on hi/lo parts), P.V on v_mfma_f32_16x16x4_f32.
//
// Workgroup: 16 queries (a query tile) x HG of the G query heads of one KV
// head, two waves per head, each taking half of every staged 64-key block (so
// a tile's serial chain is half its keys); the 2HG waves share the key/value
// rows, staged in LDS 64 keys at a time, the next block's rows loading into
// registers while the current one is used.  G/HG workgroups share a (query
// tile, KV head): more, smaller workgroups even out the causal triangle's
// unequal tiles over the CUs.  Per query (as in the decode step):
// s_j = (q . k_j) * scale for j <= P (its position), m = max_j s_j,
// e_j = exp_approx(s_j - m) for j < (P+1) & ~7 and expf above (all expf when
// P+1 < 8), o = sum_j e_j v_j times 1/sum_j e_j (divided by the sum when
// P+1 < 8).  The polynomial exp is not multiplicative, so the max is found in
// a first pass over the keys and the scores are recomputed (bit-identically)
// in the second; the two halves' maxima, sums and P.V partials meet in LDS.
//
// q.k: q rows are scaled and split like the keys (k_prefill_khl; the query's
// exponent from its own 128 elements), and each dot is
// (hi.hi) + (hi.lo + lo.hi) over the scaled parts (the lo.lo term, at most
// 2^-22 of |q||k| per element, is left out), times 2^-(e_q + e_k), exact.
//
// Fragment layouts (D[4*(l/16)+r][l%16] lands in register r of lane l):
//  * scores S^T[key][query] = K . Q^T on 16x16x32 f16 (lane l feeds 8
//    consecutive contraction slots 8*(l/16) .. +7 of A row l%16 and of B
//    column l%16): slot i of step c in lane group g = l/16 is element
//    32g + 8c + i of the head (any pairing of the 128 elements works when A
//    and B agree), so each lane reads 32 consecutive halfs of one key row's
//    hi and lo parts and keeps 32 consecutive elements of its query;
//  * P.V on 16x16x4 f32 (lane l feeds A[l%16][l/16] and B[l/16][l%16]):
//    the scores give lane l query l%16 and keys 4g + r of the 16-key
//    block, which is exactly lane l's A fragment of O = P . V for step kk = r
//    if step kk pairs lane group g with key 4g + kk; V is read in that key
//    order, and output column d of tile t in lane l%16 is 4*(l%16) + t
//    (t < 4) or 64 + 4*(l%16) + t - 4, so every lane reads and writes
//    float4s.
// ---------------------------------------------------------------------------
constexpr uint32_t kAttnKS = 64;         // keys per LDS stage
constexpr uint32_t kAttnRS = kPHd + 4;   // padded LDS row (floats)

template <uint32_t G, uint32_t HG>
__global__ __launch_bounds__(128 * HG) __attribute__((amdgpu_waves_per_eu(HG))) void k_prefill_attn(const PrefillAttnArgs a) {
    static_assert(G % HG == 0, "head split");
    constexpr uint32_t NT = 128 * HG;
    constexpr uint32_t kLoads = kAttnKS * (kPHd / 4) / NT;  // float4 per thread per staged matrix
    static_assert(kLoads * NT == kAttnKS * (kPHd / 4), "stage/thread mismatch");
    static_assert(HG * 64 * 32 <= 2 * kAttnKS * kAttnRS, "the P.V exchange reuses the staging space");
    // [0]: key rows as fp16 hi (bytes 0..255) and lo (256..511); [1]: V rows
    __shared__ __attribute__((aligned(16))) float lkv[2][kAttnKS][kAttnRS];
    __shared__ __attribute__((aligned(16))) int lke[kAttnKS];  // the staged keys' exponents
    __shared__ int lvb[kAttnKS];                              // and their V rows' non-finite flags
    __shared__ float xmax[2][HG][16], xsum[HG][16];

    const uint32_t n_qt = (a.T + 15) / 16;
    // The first half of the grid takes the longest rows first, the second
    // half the shortest first: a CU that holds workgroups b and b + half the
    // grid then gets about the same number of keys as any other.
    const uint32_t qt = (2 * blockIdx.y < gridDim.y) ? n_qt - 1 - blockIdx.x : blockIdx.x;
    const uint32_t kvh = blockIdx.y / (G / HG), hs = blockIdx.y % (G / HG);
    const uint32_t t0 = qt * 16;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t hw = wave % HG, half = wave / HG;  // head within the workgroup, half of each block
    const uint32_t h = kvh * G + hs * HG + hw;
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t t_last = min(t0 + 15u, a.T - 1u);
    const uint32_t n_keys = a.pos0 + t_last + 1u;  // keys of the tile's last query
    const uint32_t n_stages = (n_keys + kAttnKS - 1) / kAttnKS;
    const size_t q_ld = (size_t)a.n_heads * kPHd;
    const float* kbase = a.kv + (size_t)kvh * a.max_seq * 2 * kPHd;
    // key rows (hi|lo halfs, 128 floats' worth each) and exponents
    const float* khbase = reinterpret_cast<const float*>(a.khl) + (size_t)kvh * a.max_seq * kPHd;
    const int* kmbase = khl_meta(a.khl, a.n_kv, a.max_seq) + (size_t)kvh * a.max_seq;

    // This lane's query (B column li) and its 32 elements 32*lg .. 32*lg+31.
    const uint32_t my_t = t0 + li;
    const bool q_ok = my_t < a.T;
    const uint32_t P = a.pos0 + my_t;  // attends keys 0..P
    const uint32_t S = P + 1u;
    const uint32_t Sv = S >= 8u ? (S & ~7u) : 0u;
    // Its scaled hi/lo parts, step c holding elements 32*lg + 8c .. +7, and
    // its exponent (the max over the 4 lanes that hold the query).
    h8v qh[4], ql[4];
    int eq = 0;
    {
        float qv[32];
        const float4* qr = reinterpret_cast<const float4*>(a.q + (size_t)(q_ok ? my_t : t_last) * q_ld +
                                                           (size_t)h * kPHd + 32 * lg);
        float m = 0.0f;
        bool nan = false;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 v = qr[c];
            qv[4 * c + 0] = q_ok ? v.x : 0.0f;
            qv[4 * c + 1] = q_ok ? v.y : 0.0f;
            qv[4 * c + 2] = q_ok ? v.z : 0.0f;
            qv[4 * c + 3] = q_ok ? v.w : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            m = fmaxf(m, fabsf(qv[i]));
            nan |= qv[i] != qv[i];
        }
        if (nan) m = INFINITY;  // no scaling
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        eq = split_exp(m);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float v = ldexpf(qv[8 * c + i], eq);
                const _Float16 hv = (_Float16)v;
                qh[c][i] = hv;
                ql[c][i] = (_Float16)(v - (float)hv);
            }
    }

    // Rows st*KS .. +KS-1 of K (and V): fetch into registers, then put into
    // LDS; rows past the tile's keys repeat its last key (in bounds; masked
    // by j <= P below).
    // (vectors rather than arrays: arrays live across the loop stayed in
    // scratch memory)
    typedef float stage_v __attribute__((ext_vector_type(4 * kLoads)));
    typedef int stage_e __attribute__((ext_vector_type(kLoads)));
    stage_v kr, vr;
    stage_e km;  // 2e + V flag of the rows whose float4 0 this thread holds
    // mode: 0 = K rows, 1 = K and V rows, 2 = V rows
    using NoV = std::integral_constant<int, 0>;
    using WithV = std::integral_constant<int, 1>;
    using OnlyV = std::integral_constant<int, 2>;
    auto fetch = [&](uint32_t st, auto modec) {
        constexpr int mode = decltype(modec)::value;
        constexpr bool with_k = mode != 2, with_v = mode != 0;
#pragma unroll
        for (uint32_t u = 0; u < kLoads; ++u) {
            const uint32_t i = threadIdx.x + u * NT;
            const uint32_t r = i / (kPHd / 4), c = i % (kPHd / 4);
            uint32_t j = st * kAttnKS + r;
            j = j < n_keys ? j : n_keys - 1u;
            const float4* src = reinterpret_cast<const float4*>(kbase + (size_t)j * 2 * kPHd) + c;
            if constexpr (with_k) {
                // 16 bytes of the key's hi|lo row, moved as raw bits
                const float4 k4 = reinterpret_cast<const float4*>(khbase + (size_t)j * kPHd)[c];
                kr[4 * u] = k4.x;
                kr[4 * u + 1] = k4.y;
                kr[4 * u + 2] = k4.z;
                kr[4 * u + 3] = k4.w;
            }
            if (c == 0) km[u] = kmbase[j];
            if constexpr (with_v) {
                const float4 v4 = src[kPHd / 4];
                vr[4 * u] = v4.x;
                vr[4 * u + 1] = v4.y;
                vr[4 * u + 2] = v4.z;
                vr[4 * u + 3] = v4.w;
            }
        }
    };
    auto put = [&](auto modec) {
        constexpr int mode = decltype(modec)::value;
        constexpr bool with_k = mode != 2, with_v = mode != 0;
#pragma unroll
        for (uint32_t u = 0; u < kLoads; ++u) {
            const uint32_t i = threadIdx.x + u * NT;
            const uint32_t r = i / (kPHd / 4), c = i % (kPHd / 4);
            if constexpr (with_k) {
                *reinterpret_cast<float4*>(&lkv[0][r][4 * c]) =
                    make_float4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]);
                if (c == 0) lke[r] = km[u] >> 1;
            }
            if constexpr (with_v)
                if (c == 0) lvb[r] = km[u] & 1;
            if constexpr (with_v)
                *reinterpret_cast<float4*>(&lkv[1][r][4 * c]) =
                    make_float4(vr[4 * u], vr[4 * u + 1], vr[4 * u + 2], vr[4 * u + 3]);
        }
    };

    // Scores of keys sub*16 .. sub*16+15 of the staged block (times scale
    // applied by the caller): hi.hi and the two cross terms in two chains,
    // their sum, then the exponents undone.
    auto scores = [&](uint32_t sub) -> f4v {
        f4v d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = {0.0f, 0.0f, 0.0f, 0.0f};
        const _Float16* kr = reinterpret_cast<const _Float16*>(&lkv[0][sub * 16 + li][0]) + 32 * lg;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const h8v kh = *reinterpret_cast<const h8v*>(kr + 8 * c);
            const h8v kl = *reinterpret_cast<const h8v*>(kr + kPHd + 8 * c);
            d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[c], d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[c], d1, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[c], d1, 0, 0, 0);
        }
        f4v d = d0 + d1;
        const int4 ek = *reinterpret_cast<const int4*>(&lke[sub * 16 + 4 * lg]);
        d[0] = ldexpf(d[0], -(eq + ek.x));
        d[1] = ldexpf(d[1], -(eq + ek.y));
        d[2] = ldexpf(d[2], -(eq + ek.z));
        d[3] = ldexpf(d[3], -(eq + ek.w));
        return d;
    };

    // Row max over the 16 keys of d (scores of keys jb .. jb+15).
    float mx = -INFINITY;
    auto max_sub = [&](uint32_t jb, const f4v& d) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t j = jb + 4 * lg + r;
            const float sc = d[r] * a.scale;
            if (q_ok && j <= P) mx = fmaxf(mx, sc);
        }
    };
    // Both halves' maxima, through LDS.
    auto exchange_max = [&]() {
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        if (lane < 16) xmax[half][hw][lane] = mx;
        __syncthreads();
        mx = fmaxf(xmax[0][hw][li], xmax[1][hw][li]);
    };
    // e_j of the 16 keys of d, their sum and P.V with the staged V rows.
    f4v acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    float sum = 0.0f;
    auto pv_sub = [&](uint32_t sub, uint32_t jb, const f4v& d) {
        float e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t j = jb + 4 * lg + r;
            const float dd = d[r] * a.scale - mx;
            float ev = 0.0f;
            if (q_ok && j <= P) ev = (j < Sv) ? exp_approx(dd) : expf(dd);
            e[r] = ev;
            sum += ev;
        }
        // A 16-key block whose e_j are 0 for every query of the tile adds
        // exact zeros (0 * v_j for finite v_j): its P.V is skipped.  (The
        // polynomial exp is 0 below about -2.18, so most keys of a peaked
        // score row take no part.)
        const bool nz = (e[0] != 0.0f) | (e[1] != 0.0f) | (e[2] != 0.0f) | (e[3] != 0.0f);
        if (__ballot(nz || lvb[sub * 16 + li] != 0) == 0ull) return;  // wave-uniform
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const float* vr = &lkv[1][sub * 16 + 4 * lg + kk][0];
            const float4 v0 = *reinterpret_cast<const float4*>(vr + 4 * li);
            const float4 v1 = *reinterpret_cast<const float4*>(vr + 64 + 4 * li);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v0.x, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v0.y, acc[1], 0, 0, 0);
            acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v0.z, acc[2], 0, 0, 0);
            acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v0.w, acc[3], 0, 0, 0);
            acc[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v1.x, acc[4], 0, 0, 0);
            acc[5] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v1.y, acc[5], 0, 0, 0);
            acc[6] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v1.z, acc[6], 0, 0, 0);
            acc[7] = __builtin_amdgcn_mfma_f32_16x16x4f32(e[kk], v1.w, acc[7], 0, 0, 0);
        }
    };

    constexpr uint32_t kCacheStages = 8;  // up to 512 keys: pass 1's scores stay in registers
    if (n_stages <= kCacheStages) {
        f4v sc[kCacheStages][2];
        // ---- pass 1: scores and row max ----
        fetch(0, NoV{});
#pragma unroll
        for (uint32_t st = 0; st < kCacheStages; ++st) {
            if (st < n_stages) {
                __syncthreads();  // the previous stage's reads are done
                put(NoV{});
                __syncthreads();
                if (st + 1 < n_stages) fetch(st + 1, NoV{});
#pragma unroll
                for (uint32_t s2 = 0; s2 < 2; ++s2) {
                    const uint32_t sub = 2 * half + s2;
                    const uint32_t jb = st * kAttnKS + sub * 16;
                    if (jb < n_keys) {
                        sc[st][s2] = scores(sub);
                        max_sub(jb, sc[st][s2]);
                    }
                }
            }
        }
        fetch(0, OnlyV{});  // pass 2's first block, in flight during the exchange
        exchange_max();
        // ---- pass 2: e_j, their sum and P.V (V rows only staged) ----
#pragma unroll
        for (uint32_t st = 0; st < kCacheStages; ++st) {
            if (st < n_stages) {
                __syncthreads();
                put(OnlyV{});
                __syncthreads();
                if (st + 1 < n_stages) fetch(st + 1, OnlyV{});
#pragma unroll
                for (uint32_t s2 = 0; s2 < 2; ++s2) {
                    const uint32_t sub = 2 * half + s2;
                    const uint32_t jb = st * kAttnKS + sub * 16;
                    if (jb < n_keys) pv_sub(sub, jb, sc[st][s2]);
                }
            }
        }
    } else {
        // ---- pass 1: row max (this half's keys, then both halves) ----
        fetch(0, NoV{});
        for (uint32_t st = 0; st < n_stages; ++st) {
            __syncthreads();  // the previous stage's reads are done
            put(NoV{});
            __syncthreads();
            if (st + 1 < n_stages) fetch(st + 1, NoV{});
#pragma unroll
            for (uint32_t s2 = 0; s2 < 2; ++s2) {
                const uint32_t sub = 2 * half + s2;
                const uint32_t jb = st * kAttnKS + sub * 16;
                if (jb >= n_keys) break;
                max_sub(jb, scores(sub));
            }
        }
        fetch(0, WithV{});  // pass 2's first block, in flight during the exchange
        exchange_max();
        // ---- pass 2: scores again (bit-identical), e_j, sum and P.V ----
        for (uint32_t st = 0; st < n_stages; ++st) {
            __syncthreads();
            put(WithV{});
            __syncthreads();
            if (st + 1 < n_stages) fetch(st + 1, WithV{});
#pragma unroll
            for (uint32_t s2 = 0; s2 < 2; ++s2) {
                const uint32_t sub = 2 * half + s2;
                const uint32_t jb = st * kAttnKS + sub * 16;
                if (jb >= n_keys) break;
                pv_sub(sub, jb, scores(sub));
            }
        }
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);

    // ---- the second half's partials join the first's through LDS (the
    // staging space, free after this barrier) ----
    __syncthreads();
    float* xo = &lkv[0][0][0] + (size_t)(hw * 64 + lane) * 32;
    if (half == 1) {
#pragma unroll
        for (int t = 0; t < 8; ++t) *reinterpret_cast<f4v*>(xo + 4 * t) = acc[t];
        if (lane < 16) xsum[hw][lane] = sum;
    }
    __syncthreads();
    if (half == 1) return;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] += *reinterpret_cast<const f4v*>(xo + 4 * t);
    sum += xsum[hw][li];

    // ---- output: register r of lane l is query 4*(l/16) + r ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t i = 4 * lg + (uint32_t)r;
        const float total = __shfl(sum, (int)i);  // lane i holds query i's sum
        const uint32_t t = t0 + i;
        if (t < a.T) {
            const bool small = a.pos0 + t + 1u < 8u;
            const float inv = 1.0f / total;
            float o[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] = small ? acc[c][r] / total : acc[c][r] * inv;
            float* dst = a.o + (size_t)t * q_ld + (size_t)h * kPHd;
            *reinterpret_cast<float4*>(dst + 4 * li) = make_float4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<float4*>(dst + 64 + 4 * li) = make_float4(o[4], o[5], o[6], o[7]);
        }
    }
}

template <uint32_t G>
static hipError_t run_prefill_attention(const PrefillAttnArgs& a, hipStream_t s) {
    constexpr uint32_t HG = G < 2 ? G : 2;  // heads per workgroup
    const uint32_t n_keys = a.pos0 + a.T;
    hipLaunchKernelGGL(k_prefill_khl, dim3((n_keys + 7) / 8, a.n_kv), dim3(256), 0, s, a.kv, n_keys, a.max_seq,
                       static_cast<_Float16*>(a.khl), khl_meta(a.khl, a.n_kv, a.max_seq));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t n_qt = (a.T + 15) / 16;
    hipLaunchKernelGGL((k_prefill_attn<G, HG>), dim3(n_qt, a.n_kv * (G / HG)), dim3(128 * HG), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t s) {
    if (a.T == 0 || a.n_kv == 0 || a.n_heads % a.n_kv != 0 || (uint64_t)a.pos0 + a.T > a.max_seq || !a.khl)
        return hipErrorInvalidValue;
    switch (a.n_heads / a.n_kv) {
        case 1: return run_prefill_attention<1>(a, s);
        case 2: return run_prefill_attention<2>(a, s);
        case 4: return run_prefill_attention<4>(a, s);
        case 8: return run_prefill_attention<8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qh
