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
//   3. top-k (0 < k < V): the k largest p (equal probabilities in index
//      order), their sum taken sequentially in that order, p_i /= sum inside
//      the set, 0 outside; k >= V: every token valid, p unchanged;
//   4. top-p (0 < top_p < 1): the current p in descending order (ties in
//      index order), the running fp32 sum in that order until it reaches
//      top_p (the smallest such prefix; all V if it never does), p_i /= that
//      sum inside the prefix, 0 outside; top_p >= 1: every token valid (this
//      replaces a top-k set, as in the reference);
//   5. the token: running fp32 sum over the valid tokens in index order,
//      the first with r < sum; past the end, the last valid token.
// Step 1 is applied by the softmax kernels as they read the logits, and
// step 2's final multiply by 1/sum by k_filter_draw as it reads the
// exponentials (the same operations, so the same bits).
// Steps 3-5 run in one workgroup (k_filter_draw) on the nonzero
// probabilities only: the reference's clamped polynomial exp makes all but a
// few exactly zero, and a zero is never selected before a nonzero value,
// never changes a running sum and is never drawn.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "qh_kernels.hpp"
#include "qh_sample.hpp"
#include "qh_vec.hpp"

namespace qh {

namespace {

constexpr int kThreads = 256;

// Temperature: x_i * (1/T) over the 8-wide part when the logits are 32-byte
// aligned (i < n_mul), x_i / T elsewhere (reference main.c:311-427).  The
// softmax kernels apply it to the logits as they read them.
struct Temp {
    uint32_t n_mul;
    float inv, t;
};

__device__ __forceinline__ float temp_of(const Temp& tp, const float* __restrict__ x, uint32_t i) {
    return i < tp.n_mul ? x[i] * tp.inv : x[i] / tp.t;
}

__global__ __launch_bounds__(kThreads) void k_scale_temp(const float* __restrict__ x, uint32_t V, Temp tp,
                                                       float* __restrict__ y) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) y[i] = temp_of(tp, x, i);
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

__global__ __launch_bounds__(kThreads) void k_max_part(const float* __restrict__ x, uint32_t V, Temp tp,
                                                     float* __restrict__ part, uint32_t slice) {
    __shared__ float red[kThreads / 64];
    const uint32_t b0 = blockIdx.x * slice, b1 = V - b0 > slice ? b0 + slice : V;
    float m = -INFINITY;
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += kThreads) m = fmaxf(m, temp_of(tp, x, i));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w]);
        part[blockIdx.x] = fmaxf(m, red[0]);
    }
}

__global__ __launch_bounds__(kThreads) void k_exp_elems(const float* __restrict__ x, uint32_t V, Temp tp,
                                                      const float* __restrict__ part, uint32_t G,
                                                      float* __restrict__ e) {
    float m = -INFINITY;
    for (uint32_t g = 0; g < G; ++g) m = fmaxf(m, part[g]);
    const uint32_t nv = V & ~7u;
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < V) {
        const float d = temp_of(tp, x, i) - m;
        e[i] = i < nv ? exp_approx(d) : expf(d);
    }
}

// One wave; lanes 0..7 carry the eight sums.  out[0] = 1/sum.
// Sparse form (nz = nzc[0] nonzero terms, listed in index order in nzl, at
// most kSparseTerms): only the nonzero terms are added, each to its lane's
// sum in index order.  Adding a zero to a sum that starts at +0 never
// changes it, so this is the dense sum to the bit.
// Dense form (more terms, or no list: nzl == nullptr): blocks of 512
// elements (64 groups of 8) are staged through LDS, the next block's global
// loads issued before the current block is summed.
constexpr uint32_t kSparseTerms = 4096;

__global__ __launch_bounds__(64) void k_lane_sums(const float* __restrict__ e, uint32_t V,
                                                const uint32_t* __restrict__ nzl, const uint32_t* __restrict__ nzc,
                                                float* __restrict__ out) {
    __shared__ float blk[2][512];
    const uint32_t lane = threadIdx.x;
    const uint32_t nv = V & ~7u, ng = nv / 8;  // groups of 8 in the vector part
    const uint32_t nz = nzl ? nzc[0] : 0xFFFFFFFFu;
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

// Entries at offsets >= cap are not written (a caller that only reads the
// list when it holds at most cap entries sizes it to cap).
__global__ __launch_bounds__(kThreads) void k_scatter(const float* __restrict__ p, const uint8_t* __restrict__ m,
                                                    uint32_t V, const uint32_t* __restrict__ cc,
                                                    uint32_t* __restrict__ list, uint32_t cap) {
    const uint32_t chunk = blockIdx.x;
    const uint32_t i0 = chunk * kChunk + 4 * threadIdx.x;
    uint32_t bits, last1 = 0;
    const uint32_t c = take4(p, m, V, i0, bits, last1);
    uint32_t total;
    uint32_t at = cc[chunk] + block_excl(c, &total);
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u)
        if (bits & (1u << u)) {
            if (at < cap) list[at] = i0 + u;
            ++at;
        }
}

// y_i = e_i * inv[0] (the softmax's last step, N >= 8).
__global__ __launch_bounds__(kThreads) void k_scale_inv(float* __restrict__ y, uint32_t N,
                                                      const float* __restrict__ inv) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < N) y[i] = y[i] * inv[0];
}

// Selection and draw, one workgroup (steps 3-5).  The nonzero p, in index
// order, are loaded as (index, p) entries (from the nonzero-exponential list,
// or from every index when there is none); a zero p is never selected and
// never drawn, so only these entries are sorted and walked.  Sorting uses
// 64-bit keys (p bits << 32 | ~position): descending order is p descending,
// equal p in index order.  Zero-valued tokens enter a top-k set only as its
// last members (lowest indices first); they change no sum, and they matter
// only as the fallback "last valid index", which is computed from their
// count.  Up to kSelLds entries live in LDS; more (near-flat distributions)
// run the same code on global scratch.
constexpr uint32_t kSelThreads = 1024;
constexpr uint32_t kSelLds = 4096;

struct FilterArgs {
    const float* p;          // probabilities, or the exponentials when inv is set
    const float* inv;        // null, or 1/sum: p_i = e_i * *inv (the reference's scaling, applied on read)
    uint32_t V;
    const uint32_t* cand;    // nonzero-exponential indices in index order, or null: 0..V-1
    const uint32_t* cand_n;  // their count
    uint32_t top_k;
    float top_p;
    uint32_t nucleus_all;
    float r;
    unsigned long long* gkeys;  // >= pow2(V) entries (large path)
    float* gq;                  // V
    uint32_t* gidx;             // V
    uint8_t* gvalid;            // V
    uint32_t* token;
};

constexpr uint32_t kNotReached = 0xFFFFFFFFu;

__device__ __forceinline__ uint32_t key_pos(unsigned long long k) { return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull); }

// Descending bitonic sort of n (a power of two) keys by the whole workgroup.
__device__ void bitonic_desc(unsigned long long* k, uint32_t n) {
    for (uint32_t size = 2; size <= n; size <<= 1)
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = threadIdx.x; t < n / 2; t += kSelThreads) {
                const uint32_t i = (t / stride) * 2u * stride + (t % stride), l = i + stride;
                const unsigned long long x = k[i], y = k[l];
                const bool desc = (i & size) == 0;
                if (desc ? (x < y) : (x > y)) {
                    k[i] = y;
                    k[l] = x;
                }
            }
            __syncthreads();
        }
}

// Keys of the entries with a nonzero value (others and the padding up to
// np: 0), then the sort.
__device__ void sort_nonzero(unsigned long long* K, const float* Q, uint32_t n, uint32_t np) {
    for (uint32_t pos = threadIdx.x; pos < np; pos += kSelThreads) {
        unsigned long long key = 0;
        if (pos < n) {
            const uint32_t b = __float_as_uint(Q[pos]);
            if ((b & 0x7FFFFFFFu) != 0u) key = ((unsigned long long)b << 32) | (0xFFFFFFFFu - pos);
        }
        K[pos] = key;
    }
    __syncthreads();
    bitonic_desc(K, np);
}

// Wave 0: running fp32 sum over the sorted entries in order (the first
// `limit`; the walk ends at the first zero key), with a threshold: the
// first prefix reaching it.  Results in *sum_out, *cut_out (the prefix
// length, or kNotReached).
__device__ void walk_sorted(const unsigned long long* K, const float* Q, uint32_t limit, float thr, bool use_thr,
                            float* sum_out, uint32_t* cut_out) {
    const uint32_t lane = threadIdx.x & 63;
    float sum = 0.0f;
    uint32_t cut = kNotReached;
    bool done = false;
    for (uint32_t base = 0; base < limit && !done; base += 64) {
        const uint32_t j = base + lane;
        const unsigned long long key = j < limit ? K[j] : 0ull;
        const float q = key ? Q[key_pos(key)] : 0.0f;
        const uint32_t nb = (uint32_t)__popcll(__ballot(key != 0ull));
        for (uint32_t u = 0; u < nb; ++u) {
            sum += __shfl(q, (int)u);
            if (use_thr && sum >= thr) {
                cut = base + u + 1;
                done = true;
                break;
            }
        }
        if (nb < 64) done = true;
    }
    if (lane == 0) {
        *sum_out = sum;
        *cut_out = cut;
    }
}

__global__ __launch_bounds__(kSelThreads) void k_filter_draw(FilterArgs a) {
    __shared__ unsigned long long s_keys[kSelLds];
    __shared__ float s_q[kSelLds];
    __shared__ uint32_t s_idx[kSelLds];
    __shared__ uint8_t s_valid[kSelLds];
    __shared__ uint32_t s_wcnt[kSelThreads / 64];
    __shared__ uint32_t s_red[kSelThreads / 64];
    __shared__ float s_sum;
    __shared__ uint32_t s_cut;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t V = a.V;
    const uint32_t nc = a.cand ? *a.cand_n : V;
    const bool big = nc > kSelLds;
    unsigned long long* K = big ? a.gkeys : s_keys;
    float* Q = big ? a.gq : s_q;
    uint32_t* I = big ? a.gidx : s_idx;
    uint8_t* VAL = big ? a.gvalid : s_valid;

    // nonzero entries in index order
    uint32_t n = 0;
    for (uint32_t base = 0; base < nc; base += kSelThreads) {
        const uint32_t j = base + tid;
        uint32_t i = 0;
        float v = 0.0f;
        bool take = false;
        if (j < nc) {
            i = a.cand ? a.cand[j] : j;
            v = a.p[i];
            if (a.inv) v = v * *a.inv;
            take = (__float_as_uint(v) & 0x7FFFFFFFu) != 0u;
        }
        const uint64_t bal = __ballot(take);
        const uint32_t below = (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) s_wcnt[wave] = (uint32_t)__popcll(bal);
        __syncthreads();
        uint32_t off = n, tot = 0;
        for (uint32_t w = 0; w < kSelThreads / 64; ++w) {
            if (w < wave) off += s_wcnt[w];
            tot += s_wcnt[w];
        }
        if (take) {
            I[off + below] = i;
            Q[off + below] = v;
        }
        n += tot;
        __syncthreads();
    }
    uint32_t np = 1;
    while (np < n) np <<= 1;

    // max index over the entries marked valid (all threads; result in s_red[0])
    auto max_valid_index = [&](void) -> uint32_t {
        uint32_t mx = 0;
        for (uint32_t pos = tid; pos < n; pos += kSelThreads)
            if (VAL[pos] && I[pos] > mx) mx = I[pos];
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t t = (uint32_t)__shfl_xor((int)mx, o);
            mx = t > mx ? t : mx;
        }
        if (lane == 0) s_red[wave] = mx;
        __syncthreads();
        uint32_t r = 0;
        for (uint32_t w = 0; w < kSelThreads / 64; ++w) r = s_red[w] > r ? s_red[w] : r;
        __syncthreads();
        return r;
    };
    auto renorm = [&](float sum, bool all) {
        if (sum > 0.0f)
            for (uint32_t pos = tid; pos < n; pos += kSelThreads) Q[pos] = (all || VAL[pos]) ? Q[pos] / sum : 0.0f;
        __syncthreads();
    };

    bool all_valid = false, filtered = false;
    uint32_t last = 0;
    // top-k (reference main.c:431-521)
    if (a.top_k > 0) {
        if (a.top_k >= V) {
            all_valid = true;
        } else {
            sort_nonzero(K, Q, n, np);
            const uint32_t kk = a.top_k < n ? a.top_k : n;
            if (wave == 0) walk_sorted(K, Q, kk, 0.0f, false, &s_sum, &s_cut);
            for (uint32_t pos = tid; pos < n; pos += kSelThreads) VAL[pos] = 0;
            __syncthreads();
            for (uint32_t j = tid; j < kk; j += kSelThreads) VAL[key_pos(K[j])] = 1;
            __syncthreads();
            last = max_valid_index();
            if (a.top_k > n) {
                // the (top_k - n)-th zero-valued index: the nonzero indices
                // at or below the candidate push it up by one each
                if (tid == 0) {
                    uint32_t c = a.top_k - n - 1u;
                    for (uint32_t pos = 0; pos < n && I[pos] <= c; ++pos) ++c;
                    s_cut = c;
                }
                __syncthreads();
                last = s_cut > last ? s_cut : last;
            }
            renorm(s_sum, false);
            all_valid = false;
        }
        filtered = true;
    }
    // top-p (reference main.c:720-808, 525-597)
    if (a.top_p > 0.0f) {
        if (a.top_p >= 1.0f) {
            all_valid = true;
        } else {
            sort_nonzero(K, Q, n, np);
            if (wave == 0) walk_sorted(K, Q, n, a.top_p, a.nucleus_all == 0u, &s_sum, &s_cut);
            __syncthreads();
            const float sum = s_sum;
            const uint32_t cut = s_cut;
            if (a.nucleus_all || cut == kNotReached) {
                // never reached (or not searched): the nucleus is every token
                all_valid = true;
                renorm(sum, true);
            } else {
                for (uint32_t pos = tid; pos < n; pos += kSelThreads) VAL[pos] = 0;
                __syncthreads();
                for (uint32_t j = tid; j < cut; j += kSelThreads) VAL[key_pos(K[j])] = 1;
                __syncthreads();
                last = max_valid_index();
                renorm(sum, false);
                all_valid = false;
            }
        }
        filtered = true;
    }
    if (!filtered) all_valid = true;
    if (all_valid) last = V - 1u;
    // the draw (reference main.c:811-849): running sum over the valid
    // entries in index order
    if (wave == 0) {
        float cs = 0.0f;
        uint32_t tok = last;
        bool done = false;
        for (uint32_t base = 0; base < n && !done; base += 64) {
            const uint32_t j = base + lane;
            const bool ok = j < n && (all_valid || VAL[j]);
            const float q = ok ? Q[j] : 0.0f;
            const uint32_t id = j < n ? I[j] : 0u;
            const uint32_t m = n - base < 64 ? n - base : 64;
            for (uint32_t u = 0; u < m; ++u) {
                if (!__shfl((int)ok, (int)u)) continue;
                cs += __shfl(q, (int)u);
                if (a.r < cs) {
                    tok = (uint32_t)__shfl((int)id, (int)u);
                    done = true;
                    break;
                }
            }
        }
        if (lane == 0) *a.token = tok;
    }
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
    size_t scaled, probs, list, chunks, smx, scal, gkeys, gq, gidx, gvalid, total;
};

Layout layout_of(uint32_t V) {
    Layout L{};
    size_t at = 0;
    auto carve = [&](size_t b) {
        const size_t o = at;
        at += up256(b);
        return o;
    };
    size_t p2 = 1;
    while (p2 < V) p2 <<= 1;
    L.scaled = carve((size_t)V * 4);
    L.probs = carve((size_t)V * 4);
    L.list = carve((size_t)V * 4);
    L.chunks = carve((size_t)2 * ((V + kChunk - 1) / kChunk) * 4);
    L.smx = carve((size_t)((V + kMaxSlice - 1) / kMaxSlice) * 4);
    L.scal = carve(64);
    L.gkeys = carve(p2 * 8);
    L.gq = carve((size_t)V * 4);
    L.gidx = carve((size_t)V * 4);
    L.gvalid = carve(V);
    L.total = at;
    return L;
}

}  // namespace

hipError_t launch_token_feedback(const uint32_t* tok, uint32_t* pos, uint32_t* hist, uint32_t* hist_n,
                                 uint32_t hist_cap, hipStream_t s) {
    hipLaunchKernelGGL(k_feedback, dim3(1), dim3(64), 0, s, tok, pos, hist, hist_n, hist_cap);
    return hipGetLastError();
}

size_t sample_workspace_bytes(uint32_t V) { return V == 0 ? 0 : layout_of(V).total; }

hipError_t launch_sample(const float* logits, const SampleParams& sp, void* ws, uint32_t* token, hipStream_t s) {
    const uint32_t V = sp.vocab;
    if (V == 0 || !logits || !ws || !token) return hipErrorInvalidValue;
    const Layout L = layout_of(V);
    uint8_t* W = static_cast<uint8_t*>(ws);
    float* scaled = reinterpret_cast<float*>(W + L.scaled);
    float* probs = reinterpret_cast<float*>(W + L.probs);
    uint32_t* list = reinterpret_cast<uint32_t*>(W + L.list);
    uint32_t* chunks = reinterpret_cast<uint32_t*>(W + L.chunks);
    float* smx = reinterpret_cast<float*>(W + L.smx);
    float* scal = reinterpret_cast<float*>(W + L.scal);  // [6] 1/sum, [8,9] nonzero exponentials
    const dim3 grid((V + kThreads - 1) / kThreads);
    hipError_t e;
#define QH_K(...)                                            \
    do {                                                     \
        hipLaunchKernelGGL(__VA_ARGS__);                     \
        if ((e = hipGetLastError()) != hipSuccess) return e; \
    } while (0)

    // 1-2: temperature and softmax; the nonzero exponentials are listed in
    // index order for the sums and the selection
    const Temp tp{sp.n_mul, sp.inv_temperature, sp.temperature};
    FilterArgs fa{};
    if (V < 8) {
        QH_K(k_scale_temp, grid, dim3(kThreads), 0, s, logits, V, tp, scaled);
        QH_K(k_softmax_small, dim3(1), dim3(64), 0, s, scaled, V, probs);
        fa.cand = nullptr;
        fa.cand_n = nullptr;
    } else {
        const uint32_t G = (V + kMaxSlice - 1) / kMaxSlice;
        QH_K(k_max_part, dim3(G), dim3(kThreads), 0, s, logits, V, tp, smx, kMaxSlice);
        QH_K(k_exp_elems, grid, dim3(kThreads), 0, s, logits, V, tp, smx, G, probs);
        const uint32_t nch = (V + kChunk - 1) / kChunk;
        uint32_t* nzc = reinterpret_cast<uint32_t*>(scal + 8);
        QH_K(k_count, dim3(nch), dim3(kThreads), 0, s, probs, (const uint8_t*)nullptr, V, chunks, nch);
        QH_K(k_scan_chunks, dim3(1), dim3(kThreads), 0, s, chunks, nch, nzc);
        QH_K(k_scatter, dim3(nch), dim3(kThreads), 0, s, probs, (const uint8_t*)nullptr, V, chunks, list, V);
        QH_K(k_lane_sums, dim3(1), dim3(64), 0, s, probs, V, (const uint32_t*)list, (const uint32_t*)nzc, scal + 6);
        fa.inv = scal + 6;  // the filter scales the exponentials as it reads them
        fa.cand = list;
        fa.cand_n = nzc;
    }
    // 3-5: top-k, top-p, the draw
    fa.p = probs;
    fa.V = V;
    fa.top_k = sp.top_k;
    fa.top_p = sp.top_p;
    fa.nucleus_all = sp.nucleus_all ? 1u : 0u;
    fa.r = sp.r;
    fa.gkeys = reinterpret_cast<unsigned long long*>(W + L.gkeys);
    fa.gq = reinterpret_cast<float*>(W + L.gq);
    fa.gidx = reinterpret_cast<uint32_t*>(W + L.gidx);
    fa.gvalid = W + L.gvalid;
    fa.token = token;
    QH_K(k_filter_draw, dim3(1), dim3(kSelThreads), 0, s, fa);
#undef QH_K
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// Softmax in q_softmax_f32_avx2's exact order (reference src/ops/avx2/
// softmax.c:17-132): the sampler's steps 2 without a temperature.  N < 8:
// the one-workgroup kernel's scalar path (libm-style expf, sequential sum,
// e / sum).  N >= 8: slice maxima, e_i = exp_approx(x_i - m) below N & ~7
// and expf above (written to y), the nonzero e_i listed in index order
// when the workspace holds the list, the eight lane sums and tree of
// k_lane_sums (sparse over the list when it holds at most kSparseTerms
// entries, dense otherwise), then y_i *= 1 / sum.
// Workspace: [parts: G floats][scal: 16 words][chunk counts: 2 nch words]
// [list: min(N, kSparseTerms) words]; without room for the last two the
// sums run dense.
namespace {

struct SmxExactLayout {
    uint32_t slice, G, nch;
    size_t parts, scal, chunks, list, full, dense;
};

// Slices of kMaxSlice elements, doubled until there are at most 1024.
SmxExactLayout smx_exact_layout(uint32_t N) {
    SmxExactLayout L;
    L.slice = kMaxSlice;
    while ((N + (uint64_t)L.slice - 1) / L.slice > 1024u) L.slice *= 2;
    L.G = (uint32_t)((N + (uint64_t)L.slice - 1) / L.slice);
    L.nch = (N + kChunk - 1) / kChunk;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    L.parts = 0;
    L.scal = al((size_t)L.G * 4);
    L.chunks = L.scal + 256;
    L.dense = L.chunks;
    L.list = L.chunks + al((size_t)2 * L.nch * 4);
    L.full = L.list + al((size_t)(N < kSparseTerms ? N : kSparseTerms) * 4);
    return L;
}

}  // namespace

size_t softmax_exact_ws_bytes(uint32_t N) { return N < 8 ? 0 : smx_exact_layout(N).full; }

hipError_t launch_softmax_exact(const float* x, float* y, uint32_t N, void* ws, size_t ws_bytes, hipStream_t s) {
    if (N == 0) return hipSuccess;
    if (N < 8) return launch_softmax(x, y, N, s);
    const SmxExactLayout L = smx_exact_layout(N);
    if (!ws || ws_bytes < L.dense) return hipErrorInvalidValue;
    uint8_t* W = static_cast<uint8_t*>(ws);
    float* parts = reinterpret_cast<float*>(W + L.parts);
    float* scal = reinterpret_cast<float*>(W + L.scal);  // [0] count, [1] last, [8] 1/sum
    const bool listed = ws_bytes >= L.full;
    const Temp tp{N, 1.0f, 1.0f};  // x * 1.0f: the logits unchanged
    const dim3 grid((N + kThreads - 1) / kThreads);
    hipError_t e;
#define QH_K(...)                                            \
    do {                                                     \
        hipLaunchKernelGGL(__VA_ARGS__);                     \
        if ((e = hipGetLastError()) != hipSuccess) return e; \
    } while (0)
    QH_K(k_max_part, dim3(L.G), dim3(kThreads), 0, s, x, N, tp, parts, L.slice);
    QH_K(k_exp_elems, grid, dim3(kThreads), 0, s, x, N, tp, (const float*)parts, L.G, y);
    uint32_t* nzc = reinterpret_cast<uint32_t*>(scal);
    const uint32_t* list = nullptr;
    if (listed) {
        uint32_t* chunks = reinterpret_cast<uint32_t*>(W + L.chunks);
        uint32_t* lst = reinterpret_cast<uint32_t*>(W + L.list);
        QH_K(k_count, dim3(L.nch), dim3(kThreads), 0, s, (const float*)y, (const uint8_t*)nullptr, N, chunks, L.nch);
        QH_K(k_scan_chunks, dim3(1), dim3(kThreads), 0, s, chunks, L.nch, nzc);
        QH_K(k_scatter, dim3(L.nch), dim3(kThreads), 0, s, (const float*)y, (const uint8_t*)nullptr, N,
             (const uint32_t*)chunks, lst, kSparseTerms);
        list = lst;
    }
    QH_K(k_lane_sums, dim3(1), dim3(64), 0, s, (const float*)y, N, list, (const uint32_t*)nzc, scal + 8);
    QH_K(k_scale_inv, grid, dim3(kThreads), 0, s, y, N, (const float*)(scal + 8));
#undef QH_K
    return hipSuccess;
}

}  // namespace qh
