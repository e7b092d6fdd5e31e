// k_sample.hip -- on-device token sampling with the reference's semantics
// (reference src/main.c:311-975: compute_softmax_with_temp, apply_top_k,
// apply_top_p, sample_from_distribution).
//
// Pipeline (all on one stream, logits already on the device):
//   1. scaled_i = x_i * (1/T) below n_mul (the reference's 8-wide SIMD part
//      when the logits are 32-byte aligned), x_i / T above it;
//   2. p = softmax(scaled) with q_softmax_f32_avx2's arithmetic and summation
//      order, or for V < 8 the sampler's own scalar fallback (expf,
//      sequential sum, multiply by 1/sum, uniform if the sum is not
//      positive);
//   3. top-k (0 < k < V): the k largest p (stable descending radix sort of
//      (p, index): equal probabilities keep index order), their sum taken
//      sequentially in that order, p_i /= sum inside the set, 0 outside;
//      k >= V: every token valid, p unchanged;
//   4. top-p (0 < top_p < 1): stable descending sort of the current p, the
//      running fp32 sum in that order until it reaches top_p (the smallest
//      such prefix; all V if it never does), p_i /= that sum inside the
//      prefix, 0 outside; top_p >= 1: every token valid (this replaces a
//      top-k set, as in the reference);
//   5. the token: running fp32 sum over the valid tokens in index order,
//      the first with r < sum; past the end, the last valid token.
// The sequential fp32 sums (3, 4, 5) run in one wave, element by element
// in the reference's order; zeros are skipped where adding them cannot
// change the sum (x + 0 == x), so the chains cover only nonzero entries.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>

#include "qh_kernels.hpp"
#include "qh_sample.hpp"
#include "qh_vec.hpp"

namespace qh {

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void k_scale_temp(const float* __restrict__ x, uint32_t V, uint32_t n_mul,
                                                       float inv, float t, float* __restrict__ y) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) y[i] = i < n_mul ? x[i] * inv : x[i] / t;
}

// Scalar softmax of compute_softmax_with_temp's fallback (V < 8), one thread.
__global__ void k_softmax_small(const float* __restrict__ x, uint32_t V, float* __restrict__ p) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float mx = x[0];
    for (uint32_t i = 1; i < V; ++i)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (uint32_t i = 0; i < V; ++i) {
        const float e = expf(x[i] - mx);
        p[i] = e;
        sum += e;
    }
    if (sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (uint32_t i = 0; i < V; ++i) p[i] *= inv;
    } else {
        const float u = 1.0f / (float)V;
        for (uint32_t i = 0; i < V; ++i) p[i] = u;
    }
}

// Exact softmax for V >= 8, in q_softmax_f32_avx2's order (reference
// softmax.c): m = max; e_i = exp_approx(x_i - m) below nv = V & ~7, expf
// above; sum = eight lane sums (lane l: e_{8j+l}, j = 0, 1, ... in order)
// combined as ((s0+s4)+(s1+s5))+((s2+s6)+(s3+s7)), then the tail e_i in
// index order; p_i = e_i * (1/sum).  (The general-purpose device softmax
// sums in a tree: same values to about 1e-6, not the same bits; a sampled
// token depends on the exact running sums.)
constexpr uint32_t kMaxSlice = 4096;

__global__ __launch_bounds__(kThreads) void k_max_part(const float* __restrict__ x, uint32_t V, float* __restrict__ part) {
    __shared__ float red[kThreads / 64];
    const uint32_t b0 = blockIdx.x * kMaxSlice, b1 = b0 + kMaxSlice < V ? b0 + kMaxSlice : V;
    float m = -INFINITY;
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += kThreads) m = fmaxf(m, x[i]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w]);
        part[blockIdx.x] = fmaxf(m, red[0]);
    }
}

__global__ __launch_bounds__(kThreads) void k_exp_elems(const float* __restrict__ x, uint32_t V,
                                                      const float* __restrict__ part, uint32_t G,
                                                      float* __restrict__ e) {
    float m = -INFINITY;
    for (uint32_t g = 0; g < G; ++g) m = fmaxf(m, part[g]);
    const uint32_t nv = V & ~7u;
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) {
        const float d = x[i] - m;
        e[i] = i < nv ? exp_approx(d) : expf(d);
    }
}

// One wave; lanes 0..7 carry the eight sums.  out[0] = 1/sum.
// Sparse form (nz = nzc[0] nonzero terms, listed in index order in nzl, at
// most kSparseTerms): only the nonzero terms are added, each to its lane's
// sum in index order.  Adding a zero to a sum that starts at +0 never
// changes it, so this is the dense sum to the bit.
// Dense form: blocks of 512 elements (64 groups of 8) are staged through
// LDS, the next block's global loads issued before the current block is
// summed.
constexpr uint32_t kSparseTerms = 4096;

__global__ __launch_bounds__(64) void k_lane_sums(const float* __restrict__ e, uint32_t V,
                                                const uint32_t* __restrict__ nzl, const uint32_t* __restrict__ nzc,
                                                float* __restrict__ out) {
    __shared__ float blk[2][512];
    const uint32_t lane = threadIdx.x;
    const uint32_t nv = V & ~7u, ng = nv / 8;  // groups of 8 in the vector part
    const uint32_t nz = nzc[0];
    if (nz <= kSparseTerms) {
        float acc = 0.0f;
        for (uint32_t b = 0; b < nz; b += 64) {
            const uint32_t j = b + lane;
            const uint32_t id = j < nz ? nzl[j] : 0u;
            const float v = j < nz ? e[id] : 0.0f;
            const uint32_t m = nz - b < 64 ? nz - b : 64;
            for (uint32_t u = 0; u < m; ++u) {
                const uint32_t i = (uint32_t)__shfl((int)id, (int)u);
                const float ev = __shfl(v, (int)u);
                if (i < nv && (i & 7u) == lane) acc = acc + ev;
            }
        }
        float sl[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) sl[l] = __shfl(acc, l);
        float sum = ((sl[0] + sl[4]) + (sl[1] + sl[5])) + ((sl[2] + sl[6]) + (sl[3] + sl[7]));
        // tail terms (index >= nv) close the list, at most 7 of them
        const uint32_t t0 = nz > 7 ? nz - 7 : 0;
        for (uint32_t j = t0; j < nz; ++j) {
            const uint32_t i = nzl[j];
            if (i >= nv) sum = sum + e[i];
        }
        if (lane == 0) out[0] = 1.0f / sum;
        return;
    }
    const uint32_t nb = (ng + 63) / 64;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    auto load = [&](uint32_t k) {
        const uint32_t g = k * 64 + lane;
        if (g < ng) {
            a = *reinterpret_cast<const float4*>(e + 8 * g);
            b = *reinterpret_cast<const float4*>(e + 8 * g + 4);
        }
    };
    float acc = 0.0f;
    if (nb) load(0);
    for (uint32_t k = 0; k < nb; ++k) {
        float* s = blk[k & 1];
        *reinterpret_cast<float4*>(s + 8 * lane) = a;
        *reinterpret_cast<float4*>(s + 8 * lane + 4) = b;
        if (k + 1 < nb) load(k + 1);
        __syncthreads();
        if (lane < 8) {
            const uint32_t jn = ng - k * 64 < 64 ? ng - k * 64 : 64;
#pragma unroll 16
            for (uint32_t j = 0; j < jn; ++j) acc = acc + s[8 * j + lane];
        }
    }
    float sl[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) sl[l] = __shfl(acc, l);
    float sum = ((sl[0] + sl[4]) + (sl[1] + sl[5])) + ((sl[2] + sl[6]) + (sl[3] + sl[7]));
    for (uint32_t i = nv; i < V; ++i) sum = sum + e[i];
    if (lane == 0) out[0] = 1.0f / sum;
}

__global__ __launch_bounds__(kThreads) void k_scale_by(float* __restrict__ p, uint32_t V, const float* __restrict__ inv) {
    const float s = *inv;
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) p[i] = p[i] * s;
}

// Sort keys: the bit pattern of p (p >= 0 orders as an unsigned integer;
// -0.0 is folded onto +0.0 so that all zeros tie), values: the index.
__global__ __launch_bounds__(kThreads) void k_keys(const float* __restrict__ p, uint32_t V, uint32_t* __restrict__ keys,
                                                 uint32_t* __restrict__ idx) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) {
        const uint32_t b = __float_as_uint(p[i]);
        keys[i] = b == 0x80000000u ? 0u : b;
        idx[i] = i;
    }
}

__global__ __launch_bounds__(kThreads) void k_fill_u8(uint8_t* __restrict__ m, uint32_t V, uint8_t v) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) m[i] = v;
}

// mask[idx[j]] = 1 for j < n, n = *n_dev when n_dev is given, else n_host.
__global__ __launch_bounds__(kThreads) void k_mark(const uint32_t* __restrict__ idx, uint32_t n_host,
                                                 const uint32_t* __restrict__ n_dev, uint8_t* __restrict__ m) {
    const uint32_t n = n_dev ? *n_dev : n_host;
    const uint32_t j = blockIdx.x * kThreads + threadIdx.x;
    if (j < n) m[idx[j]] = 1;
}

// p_i = mask_i ? p_i / s : 0 when s > 0 (the reference leaves p alone
// otherwise).
__global__ __launch_bounds__(kThreads) void k_renorm(float* __restrict__ p, const uint8_t* __restrict__ m, uint32_t V,
                                                   const float* __restrict__ s_dev) {
    const float s = *s_dev;
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V && s > 0.0f) p[i] = m[i] ? p[i] / s : 0.0f;
}

// One wave walks the sorted keys (descending p) in order with a running fp32
// sum: the sum of the first n entries (n = limit), or, with a threshold
// (top_p), the first prefix whose sum reaches it.  The walk stops at the
// first zero key: every later entry is zero and cannot change the sum.
//   out[0] = the sum, out[1] (as u32) = the prefix length (limit if the
//   threshold is never reached).
__global__ __launch_bounds__(64) void k_sorted_walk(const uint32_t* __restrict__ keys, uint32_t limit, float threshold,
                                                  bool use_threshold, float* __restrict__ out) {
    const uint32_t lane = threadIdx.x;
    float sum = 0.0f;
    uint32_t cut = limit;
    bool done = false;
    for (uint32_t base = 0; base < limit && !done; base += 64) {
        const uint32_t j = base + lane;
        const float v = j < limit ? __uint_as_float(keys[j]) : 0.0f;
        const uint64_t nz = __ballot(v != 0.0f && j < limit);
        const uint32_t n = (uint32_t)__popcll(nz);
        // Entries past the first zero are zero (sorted descending): the
        // nonzero ones of this batch are its first n lanes.
        for (uint32_t u = 0; u < n; ++u) {
            sum += __shfl(v, (int)u);
            if (use_threshold && sum >= threshold) {
                cut = base + u + 1;
                done = true;
                break;
            }
        }
        if (n < 64) done = true;
    }
    if (lane == 0) {
        out[0] = sum;
        out[1] = __uint_as_float(cut);
    }
}

// Valid tokens with nonzero p, in index order (list), their count and the
// last valid index (a null mask: every token valid): three parallel passes
// over chunks of kChunk elements
// (thread t of a chunk owns elements 4t .. 4t+3, so thread order is index
// order).  k_count: per-chunk count and last valid index + 1;
// k_scan_chunks (one workgroup): exclusive offsets, total, last valid;
// k_scatter: each chunk writes its entries at its offset.
constexpr uint32_t kChunk = 4 * kThreads;

__device__ __forceinline__ uint32_t take4(const float* p, const uint8_t* m, uint32_t V, uint32_t i0, uint32_t& bits,
                                          uint32_t& last1) {
    uint32_t c = 0;
    bits = 0;
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
        const uint32_t i = i0 + u;
        const bool valid = i < V && (!m || m[i] != 0);
        if (valid) last1 = i + 1;
        if (valid && p[i] != 0.0f) {
            bits |= 1u << u;
            ++c;
        }
    }
    return c;
}

// Exclusive prefix of v over the workgroup's threads (tid order); *total.
__device__ __forceinline__ uint32_t block_excl(uint32_t v, uint32_t* total) {
    __shared__ uint32_t wsum[kThreads / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)x, o);
        if (lane >= (uint32_t)o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    uint32_t off = 0, tot = 0;
    for (uint32_t w = 0; w < kThreads / 64; ++w) {
        if (w < wave) off += wsum[w];
        tot += wsum[w];
    }
    __syncthreads();
    *total = tot;
    return off + x - v;
}

__global__ __launch_bounds__(kThreads) void k_count(const float* __restrict__ p, const uint8_t* __restrict__ m,
                                                  uint32_t V, uint32_t* __restrict__ cc /* [2][nchunks] */,
                                                  uint32_t nchunks) {
    const uint32_t chunk = blockIdx.x;
    uint32_t bits, last1 = 0;
    const uint32_t c = take4(p, m, V, chunk * kChunk + 4 * threadIdx.x, bits, last1);
    uint32_t total;
    (void)block_excl(c, &total);
    __shared__ uint32_t wl[kThreads / 64];
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t t = (uint32_t)__shfl_xor((int)last1, o);
        last1 = t > last1 ? t : last1;
    }
    if ((threadIdx.x & 63) == 0) wl[threadIdx.x >> 6] = last1;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t l = 0;
        for (uint32_t w = 0; w < kThreads / 64; ++w) l = wl[w] > l ? wl[w] : l;
        cc[chunk] = total;
        cc[nchunks + chunk] = l;
    }
}

// out[0] = count, out[1] = last valid index + 1 (0: none); cc[chunk]
// becomes the chunk's exclusive offset.
__global__ __launch_bounds__(kThreads) void k_scan_chunks(uint32_t* __restrict__ cc, uint32_t nchunks,
                                                        uint32_t* __restrict__ out) {
    uint32_t carry = 0, last1 = 0;
    for (uint32_t base = 0; base < nchunks; base += kThreads) {
        const uint32_t c = base + threadIdx.x;
        const uint32_t v = c < nchunks ? cc[c] : 0u;
        const uint32_t l = c < nchunks ? cc[nchunks + c] : 0u;
        last1 = l > last1 ? l : last1;
        uint32_t total;
        const uint32_t ex = block_excl(v, &total);
        if (c < nchunks) cc[c] = carry + ex;
        carry += total;
    }
    __shared__ uint32_t wl[kThreads / 64];
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t t = (uint32_t)__shfl_xor((int)last1, o);
        last1 = t > last1 ? t : last1;
    }
    if ((threadIdx.x & 63) == 0) wl[threadIdx.x >> 6] = last1;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t l = 0;
        for (uint32_t w = 0; w < kThreads / 64; ++w) l = wl[w] > l ? wl[w] : l;
        out[0] = carry;
        out[1] = l;
    }
}

__global__ __launch_bounds__(kThreads) void k_scatter(const float* __restrict__ p, const uint8_t* __restrict__ m,
                                                    uint32_t V, const uint32_t* __restrict__ cc,
                                                    uint32_t* __restrict__ list) {
    const uint32_t chunk = blockIdx.x;
    const uint32_t i0 = chunk * kChunk + 4 * threadIdx.x;
    uint32_t bits, last1 = 0;
    const uint32_t c = take4(p, m, V, i0, bits, last1);
    uint32_t total;
    uint32_t at = cc[chunk] + block_excl(c, &total);
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u)
        if (bits & (1u << u)) list[at++] = i0 + u;
}

// The token: running fp32 sum over list (index order), first with r < sum;
// otherwise the last valid index, or V - 1 when none is valid.
__global__ __launch_bounds__(64) void k_pick(const float* __restrict__ p, const uint32_t* __restrict__ list,
                                           const uint32_t* __restrict__ cnt, uint32_t V, float r,
                                           uint32_t* __restrict__ token) {
    const uint32_t lane = threadIdx.x;
    const uint32_t n = cnt[0], last1 = cnt[1];
    float sum = 0.0f;
    uint32_t tok = last1 ? last1 - 1u : V - 1u;
    bool done = false;
    for (uint32_t base = 0; base < n && !done; base += 64) {
        const uint32_t j = base + lane;
        const uint32_t id = j < n ? list[j] : 0u;
        const float v = j < n ? p[id] : 0.0f;
        const uint32_t m = n - base < 64 ? n - base : 64;
        for (uint32_t u = 0; u < m; ++u) {
            sum += __shfl(v, (int)u);
            if (r < sum) {
                tok = (uint32_t)__shfl((int)id, (int)u);
                done = true;
                break;
            }
        }
    }
    if (lane == 0) *token = tok;
}

// Generation feedback after a sampled token: append it to the history and
// advance the position (the sampled token itself is already in *tok).
__global__ void k_feedback(const uint32_t* __restrict__ tok, uint32_t* __restrict__ pos, uint32_t* __restrict__ hist,
                           uint32_t* __restrict__ hist_n, uint32_t hist_cap) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const uint32_t n = *hist_n;
    if (n < hist_cap) hist[n] = *tok;
    *hist_n = n + 1u;
    *pos += 1u;
}

inline size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

struct Layout {
    size_t scaled, probs, keys, idx, keys2, idx2, mask, list, chunks, smx, scal, sort_tmp, total;
    size_t sort_bytes;
};

hipError_t layout_of(uint32_t V, Layout* L) {
    size_t tmp = 0;
    hipError_t e = rocprim::radix_sort_pairs_desc(nullptr, tmp, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                                  (const uint32_t*)nullptr, (uint32_t*)nullptr, V, 0, 32);
    if (e != hipSuccess) return e;
    size_t at = 0;
    auto carve = [&](size_t b) {
        const size_t o = at;
        at += up256(b);
        return o;
    };
    L->scaled = carve((size_t)V * 4);
    L->probs = carve((size_t)V * 4);
    L->keys = carve((size_t)V * 4);
    L->idx = carve((size_t)V * 4);
    L->keys2 = carve((size_t)V * 4);
    L->idx2 = carve((size_t)V * 4);
    L->mask = carve(V);
    L->list = carve((size_t)V * 4);
    L->chunks = carve((size_t)2 * ((V + kChunk - 1) / kChunk) * 4);
    L->smx = carve((size_t)((V + kMaxSlice - 1) / kMaxSlice) * 4);
    L->scal = carve(64);
    L->sort_bytes = tmp;
    L->sort_tmp = carve(tmp ? tmp : 1);
    L->total = at;
    return hipSuccess;
}

}  // namespace

hipError_t launch_token_feedback(const uint32_t* tok, uint32_t* pos, uint32_t* hist, uint32_t* hist_n,
                                 uint32_t hist_cap, hipStream_t s) {
    hipLaunchKernelGGL(k_feedback, dim3(1), dim3(64), 0, s, tok, pos, hist, hist_n, hist_cap);
    return hipGetLastError();
}

size_t sample_workspace_bytes(uint32_t V) {
    Layout L{};
    if (V == 0 || layout_of(V, &L) != hipSuccess) return 0;
    return L.total;
}

hipError_t launch_sample(const float* logits, const SampleParams& sp, void* ws, uint32_t* token, hipStream_t s) {
    const uint32_t V = sp.vocab;
    if (V == 0 || !logits || !ws || !token) return hipErrorInvalidValue;
    Layout L{};
    hipError_t e = layout_of(V, &L);
    if (e != hipSuccess) return e;
    uint8_t* W = static_cast<uint8_t*>(ws);
    float* scaled = reinterpret_cast<float*>(W + L.scaled);
    float* probs = reinterpret_cast<float*>(W + L.probs);
    uint32_t* keys = reinterpret_cast<uint32_t*>(W + L.keys);
    uint32_t* idx = reinterpret_cast<uint32_t*>(W + L.idx);
    uint32_t* keys2 = reinterpret_cast<uint32_t*>(W + L.keys2);
    uint32_t* idx2 = reinterpret_cast<uint32_t*>(W + L.idx2);
    uint8_t* mask = W + L.mask;
    uint32_t* list = reinterpret_cast<uint32_t*>(W + L.list);
    uint32_t* chunks = reinterpret_cast<uint32_t*>(W + L.chunks);
    float* smx = reinterpret_cast<float*>(W + L.smx);
    float* scal = reinterpret_cast<float*>(W + L.scal);  // [0,1] top-k walk, [2,3] top-p walk, [4,5] compact,
                                                         // [6] 1/sum, [8,9] nonzero exponentials
    void* sort_tmp = W + L.sort_tmp;
    const dim3 grid((V + kThreads - 1) / kThreads);
#define QH_K(...)                                   \
    do {                                            \
        hipLaunchKernelGGL(__VA_ARGS__);            \
        if ((e = hipGetLastError()) != hipSuccess) return e; \
    } while (0)

    // 1-2: temperature and softmax
    QH_K(k_scale_temp, grid, dim3(kThreads), 0, s, logits, V, sp.n_mul, sp.inv_temperature, sp.temperature, scaled);
    if (V < 8) {
        QH_K(k_softmax_small, dim3(1), dim3(64), 0, s, scaled, V, probs);
    } else {
        const uint32_t G = (V + kMaxSlice - 1) / kMaxSlice;
        QH_K(k_max_part, dim3(G), dim3(kThreads), 0, s, scaled, V, smx);
        QH_K(k_exp_elems, grid, dim3(kThreads), 0, s, scaled, V, smx, G, probs);
        const uint32_t nch = (V + kChunk - 1) / kChunk;
        uint32_t* nzc = reinterpret_cast<uint32_t*>(scal + 8);
        QH_K(k_count, dim3(nch), dim3(kThreads), 0, s, probs, (const uint8_t*)nullptr, V, chunks, nch);
        QH_K(k_scan_chunks, dim3(1), dim3(kThreads), 0, s, chunks, nch, nzc);
        QH_K(k_scatter, dim3(nch), dim3(kThreads), 0, s, probs, (const uint8_t*)nullptr, V, chunks, list);
        QH_K(k_lane_sums, dim3(1), dim3(64), 0, s, probs, V, (const uint32_t*)list, (const uint32_t*)nzc, scal + 6);
        QH_K(k_scale_by, grid, dim3(kThreads), 0, s, probs, V, scal + 6);
    }
    auto sort_desc = [&](void) -> hipError_t {
        size_t tb = L.sort_bytes;
        QH_K(k_keys, grid, dim3(kThreads), 0, s, probs, V, keys, idx);
        return rocprim::radix_sort_pairs_desc(sort_tmp, tb, static_cast<const uint32_t*>(keys), keys2,
                                              static_cast<const uint32_t*>(idx), idx2, V, 0, 32, s);
    };
    bool mask_set = false;
    // 3: top-k
    if (sp.top_k > 0) {
        if (sp.top_k >= V) {
            QH_K(k_fill_u8, grid, dim3(kThreads), 0, s, mask, V, (uint8_t)1);
        } else {
            if ((e = sort_desc()) != hipSuccess) return e;
            QH_K(k_sorted_walk, dim3(1), dim3(64), 0, s, keys2, sp.top_k, 0.0f, false, scal);
            QH_K(k_fill_u8, grid, dim3(kThreads), 0, s, mask, V, (uint8_t)0);
            QH_K(k_mark, dim3((sp.top_k + kThreads - 1) / kThreads), dim3(kThreads), 0, s, idx2, sp.top_k,
                 (const uint32_t*)nullptr, mask);
            QH_K(k_renorm, grid, dim3(kThreads), 0, s, probs, mask, V, scal);
        }
        mask_set = true;
    }
    // 4: top-p
    if (sp.top_p > 0.0f) {
        if (sp.top_p >= 1.0f) {
            QH_K(k_fill_u8, grid, dim3(kThreads), 0, s, mask, V, (uint8_t)1);
        } else {
            if ((e = sort_desc()) != hipSuccess) return e;
            // nucleus_all: the reference's prefix-sum buffer could not be
            // allocated; its search then keeps every token.
            QH_K(k_sorted_walk, dim3(1), dim3(64), 0, s, keys2, V, sp.top_p, !sp.nucleus_all, scal + 2);
            QH_K(k_fill_u8, grid, dim3(kThreads), 0, s, mask, V, (uint8_t)0);
            QH_K(k_mark, grid, dim3(kThreads), 0, s, idx2, V, reinterpret_cast<const uint32_t*>(scal + 3), mask);
            QH_K(k_renorm, grid, dim3(kThreads), 0, s, probs, mask, V, scal + 2);
        }
        mask_set = true;
    }
    // Neither filter: every token valid.
    if (!mask_set) QH_K(k_fill_u8, grid, dim3(kThreads), 0, s, mask, V, (uint8_t)1);
    // 5: the token
    uint32_t* cnt = reinterpret_cast<uint32_t*>(scal + 4);
    const uint32_t nchunks = (V + kChunk - 1) / kChunk;
    QH_K(k_count, dim3(nchunks), dim3(kThreads), 0, s, probs, mask, V, chunks, nchunks);
    QH_K(k_scan_chunks, dim3(1), dim3(kThreads), 0, s, chunks, nchunks, cnt);
    QH_K(k_scatter, dim3(nchunks), dim3(kThreads), 0, s, probs, mask, V, chunks, list);
    QH_K(k_pick, dim3(1), dim3(64), 0, s, probs, list, cnt, V, sp.r, token);
#undef QH_K
    return hipSuccess;
}

}  // namespace qh
