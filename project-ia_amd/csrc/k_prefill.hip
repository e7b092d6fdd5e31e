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
// Keys and values as fp16 hi/lo parts for the attention's matrix-core
// products (one layer's worth, rebuilt for every prefill chunk).
//  * Keys: row j of KV head h (keys 0 .. n_keys-1) is scaled by 2^e, e
//    chosen per row so that max|k'| lies in [2^14, 2^15) (e = 0 for an
//    all-zero or non-finite row), and split as hi = rn(k'), lo = rn(k' - hi)
//    (the subtraction is exact in fp32): 22 significant bits of every
//    element within 2^17 of the row maximum, steps of 2^-24 (of k') below
//    that.  With each row goes a flag: the key's V row holds a NaN or an
//    infinity (its P.V terms must then be formed even where e_j = 0, as
//    0 * v_j is NaN).
//  * Values: one exponent per KV head, from the largest finite |v| over its
//    keys (so that max|v'| lies in [2^14, 2^15)), the same hi/lo split, and
//    stored transposed per 64-key stage, [dim][64 keys], the keys of each
//    32-key half in the order the P.V fragments read them (positions
//    8g + 4s + r hold key 16s + 4g + r).
// Layout (256-byte aligned pieces): K halfs [n_kv][max_seq][hi 128 | lo
// 128]; int32 2e + flag [n_kv][max_seq]; float partial max|v| [n_kv]
// [max_seq / 8]; int32 V exponent [n_kv]; V halfs [n_kv][stages][hi | lo]
// [128][64].
// ---------------------------------------------------------------------------
struct KhlLayout {
    size_t meta, vmax, vexp, vt, bytes;
    uint32_t n_wa, n_st;  // partials per head (8 keys each), 64-key stages per head
};

__host__ __device__ inline KhlLayout khl_layout(uint32_t n_kv, uint32_t max_seq) {
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    KhlLayout L;
    const size_t rows = (size_t)n_kv * max_seq;
    L.n_wa = (max_seq + 7) / 8;
    L.n_st = (max_seq + 63) / 64;
    L.meta = al(rows * 2 * kPHd * 2);
    L.vmax = L.meta + al(rows * 4);
    L.vexp = L.vmax + al((size_t)n_kv * L.n_wa * 4);
    L.vt = L.vexp + al((size_t)n_kv * 4);
    L.bytes = L.vt + (size_t)n_kv * L.n_st * 64 * 2 * kPHd * 2;
    return L;
}

size_t prefill_khl_bytes(uint32_t n_kv, uint32_t max_seq) { return khl_layout(n_kv, max_seq).bytes; }

template <typename T>
__host__ __device__ inline T* khl_at(void* khl, size_t off) {
    return reinterpret_cast<T*>(static_cast<uint8_t*>(khl) + off);
}

// Exponent e with max|x * 2^e| in [2^14, 2^15) for a finite m = max|x| > 0,
// else 0.
__device__ __forceinline__ int split_exp(float m) {
    return (m > 0.0f && m <= FLT_MAX) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
}

// Key rows, their flags, and each 8-row group's largest finite |v|: one
// 32-lane half of a wave per row, one float4 of K and of V per lane.
__global__ __launch_bounds__(256) void k_prefill_khl(const float* __restrict__ kv, uint32_t n_keys, uint32_t max_seq,
                                                     void* __restrict__ khl, KhlLayout L) {
    __shared__ float red[4];
    const uint32_t kvh = blockIdx.y;
    const uint32_t j = blockIdx.x * 8u + (threadIdx.x >> 5), c = threadIdx.x & 31u;
    const bool ok = j < n_keys;  // uniform over the row's 32 lanes
    const size_t row = (size_t)kvh * max_seq + (ok ? j : 0u);
    float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f), vx = x;
    if (ok) {
        x = *reinterpret_cast<const float4*>(kv + row * (2 * kPHd) + 4 * c);
        vx = *reinterpret_cast<const float4*>(kv + row * (2 * kPHd) + kPHd + 4 * c);
    }
    const float va[4] = {fabsf(vx.x), fabsf(vx.y), fabsf(vx.z), fabsf(vx.w)};
    bool vbad = false;
    float mv = 0.0f;  // largest finite |v|
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool fin = va[i] <= FLT_MAX;
        vbad |= !fin;
        mv = fin ? fmaxf(mv, va[i]) : mv;
    }
    const uint64_t vb = __ballot(vbad);
    const bool row_vbad = ((threadIdx.x & 32) ? (uint32_t)(vb >> 32) : (uint32_t)vb) != 0u;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) mv = fmaxf(mv, __shfl_xor(mv, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mv;
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
    if (ok) {
        _Float16* dst = khl_at<_Float16>(khl, 0) + row * (2 * kPHd) + 4 * c;
        *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(hi);
        *reinterpret_cast<uint2*>(dst + kPHd) = *reinterpret_cast<const uint2*>(lo);
        if (c == 0) khl_at<int>(khl, L.meta)[row] = 2 * e + (row_vbad ? 1 : 0);
    }
    __syncthreads();
    if (threadIdx.x == 0)
        khl_at<float>(khl, L.vmax)[(size_t)kvh * L.n_wa + blockIdx.x] =
            fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Position of key r (0..63) of a stage in the transposed V rows.
__device__ __forceinline__ uint32_t vt_pos(uint32_t r) {
    const uint32_t k = r & 31u;
    return (r & 32u) + 8u * ((k >> 2) & 3u) + 4u * (k >> 4) + (k & 3u);
}

// V of one 64-key stage of one KV head, scaled by the head's exponent,
// split into hi/lo and transposed (through LDS); keys past n_keys are 0.
__global__ __launch_bounds__(256) void k_prefill_vt(const float* __restrict__ kv, uint32_t n_keys, uint32_t max_seq,
                                                    void* __restrict__ khl, KhlLayout L) {
    __shared__ float red[4];
    __shared__ __attribute__((aligned(16))) _Float16 lt[2][kPHd][64 + 8];
    const uint32_t st = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    // The head's largest finite |v| from k_prefill_khl's partials (exact, so
    // any order): every workgroup of the head gets the same exponent.
    const float* vm = khl_at<float>(khl, L.vmax) + (size_t)kvh * L.n_wa;
    const uint32_t nw = (n_keys + 7) / 8;
    float m = 0.0f;
    for (uint32_t i = tid; i < nw; i += 256) m = fmaxf(m, vm[i]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const int ev = split_exp(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    if (st == 0 && tid == 0) khl_at<int>(khl, L.vexp)[kvh] = ev;
    const float* vbase = kv + (size_t)kvh * max_seq * 2 * kPHd + kPHd;
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
        const uint32_t i = tid + 256u * u, r = i >> 5, c = i & 31u;
        const uint32_t j = st * 64u + r;
        float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (j < n_keys) x = *reinterpret_cast<const float4*>(vbase + (size_t)j * 2 * kPHd + 4 * c);
        const float xs[4] = {x.x, x.y, x.z, x.w};
        const uint32_t pos = vt_pos(r);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = ldexpf(xs[e], ev);
            const _Float16 hv = (_Float16)v;
            lt[0][4 * c + e][pos] = hv;
            lt[1][4 * c + e][pos] = (_Float16)(v - (float)hv);
        }
    }
    __syncthreads();
    _Float16* dst = khl_at<_Float16>(khl, L.vt) + ((size_t)kvh * L.n_st + st) * (2 * kPHd * 64);
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
        const uint32_t q = tid + 256u * u, part = q >> 10, d = (q >> 3) & 127u, k8 = q & 7u;
        *reinterpret_cast<uint4*>(dst + ((size_t)part * kPHd + d) * 64 + 8 * k8) =
            *reinterpret_cast<const uint4*>(&lt[part][d][8 * k8]);
    }
}

// ---------------------------------------------------------------------------
// Causal prefill attention: q.k and P.V on fp16 matrix cores
// (v_mfma_f32_16x16x32_f16 on hi/lo parts).
//
// Workgroup: 16 queries (a query tile) x HG of the G query heads of one KV
// head, two waves per head, each taking half of every staged 64-key block (so
// a tile's serial chain is half its keys); the 2HG waves share the key/value
// rows, staged in LDS 64 keys at a time, the next block's rows loading into
// registers while the current one is used.  HG = min(G, 4): a GQA group of
// up to 4 heads shares one staging of its keys and values (8 waves, one
// workgroup per CU); G = 8 takes two workgroups per (query tile, KV head).
// Workgroups start longest tile first (see the grid order below).  Per
// query (as in the decode step):
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
// P.V: e_j (at most 1 for finite scores; the reference's exp gives 91.4 for
// a NaN) times 2^9, split the same way, against the head's scaled V parts
// (k_prefill_vt): hi.hi + hi.lo + lo.hi, times 2^-(9 + e_v) at the end.
//
// Fragment layouts (D[4*(l/16)+r][l%16] lands in register r of lane l):
//  * scores S^T[key][query] = K . Q^T on 16x16x32 f16 (lane l feeds 8
//    consecutive contraction slots 8*(l/16) .. +7 of A row l%16 and of B
//    column l%16): slot i of step c in lane group g = l/16 is element
//    32g + 8c + i of the head (any pairing of the 128 elements works when A
//    and B agree), so each lane reads 32 consecutive halfs of one key row's
//    hi and lo parts and keeps 32 consecutive elements of its query;
//  * P.V on 16x16x32 f16, one MFMA step per 32 keys (a wave's half of a
//    staged block): the scores give lane l query l%16 and keys 4g + r of
//    each 16-key block, so its A row (query l%16) takes slots 8g .. 8g+3
//    from the first block and 8g+4 .. 8g+7 from the second; the transposed
//    V rows hold the keys in that slot order, so B column c of tile n
//    (dimension 16n + c) is one 16-byte read per part, and register r of
//    lane l holds query 4g + r, dimension 16n + l%16.
// ---------------------------------------------------------------------------
constexpr uint32_t kAttnKS = 64;         // keys per LDS stage
constexpr int kAttnBufFlags = 0x00020000;  // raw buffer resource word 3 (gfx9 family): out of range reads 0
typedef uint32_t u4v_a __attribute__((ext_vector_type(4)));
constexpr uint32_t kAttnRS = kPHd + 4;   // padded LDS row (floats)

template <uint32_t G, uint32_t HG>
__global__ __launch_bounds__(128 * HG) __attribute__((amdgpu_waves_per_eu(HG < 2 ? HG : 2))) void k_prefill_attn(const PrefillAttnArgs a) {
    static_assert(G % HG == 0, "head split");
    constexpr uint32_t NT = 128 * HG;
    constexpr uint32_t kLoads = kAttnKS * (kPHd / 4) / NT;  // float4 per thread per staged matrix
    static_assert(kLoads * NT == kAttnKS * (kPHd / 4), "stage/thread mismatch");
    static_assert(HG * 64 * 32 <= kAttnKS * kAttnRS, "the P.V exchange reuses the key staging space");
    // key rows as fp16 hi (bytes 0..255) and lo (256..511)
    __shared__ __attribute__((aligned(16))) float lk[kAttnKS][kAttnRS];
    // V of the staged keys, transposed: [hi | lo][dimension][key position]
    __shared__ __attribute__((aligned(16))) _Float16 lvt[2][kPHd][kAttnKS + 8];
    __shared__ __attribute__((aligned(16))) int lke[kAttnKS];  // the staged keys' exponents
    __shared__ int lvb[kAttnKS];                              // and their V rows' non-finite flags
    __shared__ float xmax[2][HG][16], xsum[HG][16];

    const uint32_t n_qt = (a.T + 15) / 16;
    // Longest query tiles first: the grid's y runs over the query tiles from
    // the last (most keys) down, x over the KV heads and head groups, so
    // workgroups start in order of decreasing work and the short tiles fill
    // the last rounds.
    const uint32_t qt = n_qt - 1 - blockIdx.y;
    const uint32_t kvh = blockIdx.x / (G / HG), hs = blockIdx.x % (G / HG);
    const uint32_t t0 = qt * 16;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t hw = wave % HG, half = wave / HG;  // head within the workgroup, half of each block
    const uint32_t h = kvh * G + hs * HG + hw;
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t t_last = min(t0 + 15u, a.T - 1u);
    const uint32_t n_keys = a.pos0 + t_last + 1u;  // keys of the tile's last query
    const uint32_t n_stages = (n_keys + kAttnKS - 1) / kAttnKS;
    const size_t q_ld = (size_t)a.n_heads * kPHd;
    const KhlLayout L = khl_layout(a.n_kv, a.max_seq);
    // key rows (hi|lo halfs, 128 floats' worth each), 2e + V flag, the
    // transposed V stages and the head's V exponent
    const float* khbase = khl_at<const float>(a.khl, 0) + (size_t)kvh * a.max_seq * kPHd;
    const int* kmbase = khl_at<const int>(a.khl, L.meta) + (size_t)kvh * a.max_seq;
    const float* vtbase = khl_at<const float>(a.khl, L.vt) + (size_t)kvh * L.n_st * (kPHd * 64);
    const int ev = khl_at<const int>(a.khl, L.vexp)[kvh];

    // This lane's query (B column li) and its 32 elements 32*lg .. 32*lg+31.
    const uint32_t my_t = t0 + li;
    const bool q_ok = my_t < a.T;
    const uint32_t P = a.pos0 + my_t;  // attends keys 0..P
    const uint32_t S = P + 1u;
    const uint32_t Sv = S >= 8u ? (S & ~7u) : 0u;
    // Keys below `inner` are attended by every query of the tile, all on the
    // polynomial exp (a full tile: the first query's Sv; 0 for a partial
    // last tile): steps of 32 keys below it need no masks.
    const uint32_t S_first = a.pos0 + t0 + 1u;
    const uint32_t inner = (t0 + 16u <= a.T && S_first >= 8u) ? (S_first & ~7u) : 0u;
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
    // LDS.  The loads go through buffer resources with per-lane offsets
    // fixed for the whole kernel and the stage as a scalar offset, so a
    // fetch costs no address arithmetic.  The K and exponent resources end
    // at the tile's last key: a valid row's lane offset always lies inside,
    // and rows past the last key (zeros, or the rows behind them in the same
    // workspace, whether or not the hardware range check counts the scalar
    // offset) only meet scores masked by j <= P below and the zero V parts
    // k_prefill_vt writes past the keys.
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
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)khbase, 0, (int)(n_keys * kPHd * 4u), kAttnBufFlags);
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc((void*)kmbase, 0, (int)(n_keys * 4u), kAttnBufFlags);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)vtbase, 0, (int)(n_stages * kPHd * 64u * 4u), kAttnBufFlags);
    // Chunk i = threadIdx.x + u*NT of a stage is bytes 16i.. of its K rows
    // (row i/32) and of its V parts alike: one lane offset, the rest scalar.
    const uint32_t lane_off = threadIdx.x * 16u, lane_row = (threadIdx.x / (kPHd / 4)) * 4u;
    auto fetch = [&](uint32_t st, auto modec) {
        constexpr int mode = decltype(modec)::value;
        constexpr bool with_k = mode != 2, with_v = mode != 0;
#pragma unroll
        for (uint32_t u = 0; u < kLoads; ++u) {
            const uint32_t so = st * (kAttnKS * kPHd * 4u) + u * NT * 16u;  // == st * 32 KB + u * NT * 16
            if constexpr (with_k) {
                // 16 bytes of the key's hi|lo row, moved as raw bits
                const u4v_a k4 = __builtin_amdgcn_raw_buffer_load_b128(rk, lane_off, so, 0);
                kr[4 * u] = __uint_as_float(k4[0]);
                kr[4 * u + 1] = __uint_as_float(k4[1]);
                kr[4 * u + 2] = __uint_as_float(k4[2]);
                kr[4 * u + 3] = __uint_as_float(k4[3]);
            }
            // every lane of the row's 32 loads its 2e + V flag (one address)
            km[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rm, lane_row, st * (kAttnKS * 4u) + u * (NT / 8u), 0);
            if constexpr (with_v) {
                // 16 bytes (chunk i) of the stage's transposed V parts, raw bits
                const u4v_a v4 = __builtin_amdgcn_raw_buffer_load_b128(rv, lane_off, so, 0);
                vr[4 * u] = __uint_as_float(v4[0]);
                vr[4 * u + 1] = __uint_as_float(v4[1]);
                vr[4 * u + 2] = __uint_as_float(v4[2]);
                vr[4 * u + 3] = __uint_as_float(v4[3]);
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
                *reinterpret_cast<float4*>(&lk[r][4 * c]) =
                    make_float4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]);
                if (c == 0) lke[r] = km[u] >> 1;
            }
            if constexpr (with_v)
                if (c == 0) lvb[r] = km[u] & 1;
            if constexpr (with_v) {
                const uint32_t part = i >> 10, d = (i >> 3) & (kPHd - 1), k8 = i & 7u;
                *reinterpret_cast<float4*>(&lvt[part][d][8 * k8]) =
                    make_float4(vr[4 * u], vr[4 * u + 1], vr[4 * u + 2], vr[4 * u + 3]);
            }
        }
    };

    // Scores of keys sub*16 .. sub*16+31 of the staged block (the wave's 32
    // keys; times scale applied by the caller), r0 for the first 16, r1 for
    // the next: per 16 keys hi.hi and the two cross terms in two chains,
    // their sum, then the exponents undone.  The two 16-key products run
    // interleaved (four independent MFMA chains).
    auto scores2 = [&](uint32_t sub, f4v& r0, f4v& r1) {
        f4v a0 = {0.0f, 0.0f, 0.0f, 0.0f}, b0 = a0, a1 = a0, b1 = a0;
        const _Float16* k0 = reinterpret_cast<const _Float16*>(&lk[sub * 16 + li][0]) + 32 * lg;
        const _Float16* k1 = reinterpret_cast<const _Float16*>(&lk[sub * 16 + 16 + li][0]) + 32 * lg;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const h8v kh0 = *reinterpret_cast<const h8v*>(k0 + 8 * c);
            const h8v kl0 = *reinterpret_cast<const h8v*>(k0 + kPHd + 8 * c);
            const h8v kh1 = *reinterpret_cast<const h8v*>(k1 + 8 * c);
            const h8v kl1 = *reinterpret_cast<const h8v*>(k1 + kPHd + 8 * c);
            a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh0, qh[c], a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh1, qh[c], a1, 0, 0, 0);
            b0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh0, ql[c], b0, 0, 0, 0);
            b1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh1, ql[c], b1, 0, 0, 0);
            b0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl0, qh[c], b0, 0, 0, 0);
            b1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl1, qh[c], b1, 0, 0, 0);
        }
        r0 = a0 + b0;
        r1 = a1 + b1;
        const int4 e0 = *reinterpret_cast<const int4*>(&lke[sub * 16 + 4 * lg]);
        const int4 e1 = *reinterpret_cast<const int4*>(&lke[sub * 16 + 16 + 4 * lg]);
        r0[0] = ldexpf(r0[0], -(eq + e0.x));
        r0[1] = ldexpf(r0[1], -(eq + e0.y));
        r0[2] = ldexpf(r0[2], -(eq + e0.z));
        r0[3] = ldexpf(r0[3], -(eq + e0.w));
        r1[0] = ldexpf(r1[0], -(eq + e1.x));
        r1[1] = ldexpf(r1[1], -(eq + e1.y));
        r1[2] = ldexpf(r1[2], -(eq + e1.z));
        r1[3] = ldexpf(r1[3], -(eq + e1.w));
    };

    // Row max over the 16 keys of d (scores of keys jb .. jb+15).
    float mx = -INFINITY;
    auto max_sub = [&](uint32_t jb, const f4v& d) {
        if (jb + 16u <= inner) {  // wave-uniform: every key attended
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, d[r] * a.scale);
            return;
        }
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
    // e_j of the wave's 32 keys (d0: keys jb .. jb+15, d1: jb+16 .. jb+31),
    // their sum and P.V with the staged V parts.
    f4v acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    float sum = 0.0f;
    auto pv32 = [&](uint32_t jb, const f4v& d0, const f4v& d1) {
        float e[8];
        if (jb + 32u <= inner) {
            // wave-uniform: every key attended, on the polynomial exp (its
            // argument s_j - m is <= 0 or NaN: exp_approx_nonpos)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int r = 0; r < 4; ++r) e[4 * s2 + r] = exp_approx_nonpos((s2 ? d1[r] : d0[r]) * a.scale - mx);
        } else {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t j = jb + 16 * s2 + 4 * lg + r;
                    const float dd = (s2 ? d1[r] : d0[r]) * a.scale - mx;
                    float ev_j = 0.0f;
                    if (q_ok && j <= P) ev_j = (j < Sv) ? exp_approx(dd) : expf(dd);
                    e[4 * s2 + r] = ev_j;
                }
        }
        // The step's 8 values summed as a tree, then added to the row sum;
        // e_j >= 0 (or NaN), so the step's values are all 0 exactly when
        // their sum is.
        const float es = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
        sum += es;
        // A 32-key step whose e_j are 0 for every query of the tile adds
        // exact zeros (0 * v_j for finite v_j): its P.V is skipped.  (The
        // polynomial exp is 0 below about -2.18, so most keys of a peaked
        // score row take no part.)
        const bool nz = es != 0.0f;
        const uint32_t kb = 32 * half;  // the wave's keys within the staged block
        if (__ballot(nz || lvb[kb + li] != 0 || lvb[kb + 16 + li] != 0) == 0ull) return;  // wave-uniform
        h8v ph, pl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = e[i] * 512.0f;
            const _Float16 hv = (_Float16)v;
            ph[i] = hv;
            pl[i] = (_Float16)(v - (float)hv);
        }
        // Four dimension tiles at a time: their 8 fragment reads first, then
        // the three products of each tile in turn across the four (the
        // same order per tile, four independent chains).
#pragma unroll
        for (int n0 = 0; n0 < 8; n0 += 4) {
            h8v vh[4], vl[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                vh[i] = *reinterpret_cast<const h8v*>(&lvt[0][16 * (n0 + i) + li][kb + 8 * lg]);
                vl[i] = *reinterpret_cast<const h8v*>(&lvt[1][16 * (n0 + i) + li][kb + 8 * lg]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[n0 + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vh[i], acc[n0 + i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[n0 + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vl[i], acc[n0 + i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[n0 + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vh[i], acc[n0 + i], 0, 0, 0);
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
                // (keys past the tile's last are masked by j <= P)
                const uint32_t jb = st * kAttnKS + 32 * half;
                scores2(2 * half, sc[st][0], sc[st][1]);
                max_sub(jb, sc[st][0]);
                max_sub(jb + 16, sc[st][1]);
            }
        }
        fetch(0, OnlyV{});  // pass 2's first block, in flight during the exchange
        exchange_max();
        // ---- pass 2: e_j, their sum and P.V (V parts only staged) ----
#pragma unroll
        for (uint32_t st = 0; st < kCacheStages; ++st) {
            if (st < n_stages) {
                __syncthreads();
                put(OnlyV{});
                __syncthreads();
                if (st + 1 < n_stages) fetch(st + 1, OnlyV{});
                const uint32_t jb = st * kAttnKS + 32 * half;
                if (jb < n_keys) pv32(jb, sc[st][0], jb + 16 < n_keys ? sc[st][1] : f4v{0.0f, 0.0f, 0.0f, 0.0f});
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
            const uint32_t jb = st * kAttnKS + 32 * half;
            f4v d0, d1;
            scores2(2 * half, d0, d1);
            max_sub(jb, d0);
            max_sub(jb + 16, d1);
        }
        fetch(0, WithV{});  // pass 2's first block, in flight during the exchange
        exchange_max();
        // ---- pass 2: scores again (bit-identical), e_j, sum and P.V ----
        for (uint32_t st = 0; st < n_stages; ++st) {
            __syncthreads();
            put(WithV{});
            __syncthreads();
            if (st + 1 < n_stages) fetch(st + 1, WithV{});
            const uint32_t jb = st * kAttnKS + 32 * half;
            if (jb < n_keys) {
                f4v d0, d1;
                scores2(2 * half, d0, d1);
                if (jb + 16 >= n_keys) d1 = f4v{0.0f, 0.0f, 0.0f, 0.0f};
                pv32(jb, d0, d1);
            }
        }
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);

    // ---- the second half's partials join the first's through LDS (the
    // staging space, free after this barrier) ----
    __syncthreads();
    float* xo = &lk[0][0] + (size_t)(hw * 64 + lane) * 32;
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

    // ---- output: register r of lane l is query 4*(l/16) + r, dimension
    // 16n + l%16 of tile n; the parts' scales undone exactly first ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t i = 4 * lg + (uint32_t)r;
        const float total = __shfl(sum, (int)i);  // lane i holds query i's sum
        const uint32_t t = t0 + i;
        if (t < a.T) {
            const bool small = a.pos0 + t + 1u < 8u;
            const float inv = 1.0f / total;
            float* dst = a.o + (size_t)t * q_ld + (size_t)h * kPHd + li;
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const float v = ldexpf(acc[n][r], -(9 + ev));
                dst[16 * n] = small ? v / total : v * inv;
            }
        }
    }
}

template <uint32_t G>
static hipError_t run_prefill_attention(const PrefillAttnArgs& a, hipStream_t s) {
    constexpr uint32_t HG = G < 4 ? G : 4;  // heads per workgroup
    const uint32_t n_keys = a.pos0 + a.T;
    const KhlLayout L = khl_layout(a.n_kv, a.max_seq);
    hipLaunchKernelGGL(k_prefill_khl, dim3((n_keys + 7) / 8, a.n_kv), dim3(256), 0, s, a.kv, n_keys, a.max_seq, a.khl,
                       L);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prefill_vt, dim3((n_keys + 63) / 64, a.n_kv), dim3(256), 0, s, a.kv, n_keys, a.max_seq,
                       a.khl, L);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t n_qt = (a.T + 15) / 16;
    hipLaunchKernelGGL((k_prefill_attn<G, HG>), dim3(a.n_kv * (G / HG), n_qt), dim3(128 * HG), 0, s, a);
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
