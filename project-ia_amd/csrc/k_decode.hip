// k_decode.hip -- decode-step kernels for gfx950 other than the GEMV:
// split-K attention over the HBM KV cache, the fused SwiGLU + digit prep,
// and the embedding row copy.
//
// Attention (corrected reference composition, model.c:1340-1440 applied to
// the cached keys 0..pos): scores s_j = dot(q_h, k_j) * scale with the dot in
// the reference's q_matmul_f32 order, softmax with the reference polynomial
// exp (libm-style expf on the N%8 tail), o_h = sum_j p_j v_j.  Because the
// polynomial exp is not multiplicative (exp_approx(a+b) != exp_approx(a) *
// exp_approx(b)), online-softmax rescaling would change results; the max is
// found first.  Three phases:
//   A  scores + per-chunk max            grid (64-key chunks, kv heads)
//   B  e_j, per-chunk sums and P.V sums  grid (256-key chunks, kv heads,
//                                        32-column slices of V)
//   C  combine + digit prep of o (the Wo GEMV input), one lane per element.
// KV layout is the reference's [L][kv_head][max_seq][K|V][head_dim].
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "qh_decode.hpp"
#include "qh_digits.hpp"
#include "qh_vec.hpp"

namespace qh {

constexpr int kHd = 128;      // head_dim this build's attention kernels are written for
constexpr int kChunk = 64;    // keys per workgroup
constexpr uint32_t kMaxGroup = 8;  // q heads per kv head (1, 2, 4 or 8)

// Reference dot order for K = 128 (matmul_fp32.c:356-425): 32 partial sums
// a[c][l] (c = 0..3 accumulators, l = 0..7 lanes), element k = 32t + 8c + l
// accumulated over t = 0..3 with FMA; S_l = (a0+a1)+(a2+a3); then
// ((S0+S4)+(S1+S5))+((S2+S6)+(S3+S7)).  Here 8 consecutive lanes compute
// one dot: lane l holds a[0..3][l], forms S_l locally, and the last tree runs
// on DPP (row_shl:4 pairs l with l+4, then quad_perm swaps 1 and 2), so the
// sum takes the reference's pairs bit for bit without LDS round trips.  The
// dot ends in lane l = 0 of each group of 8.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The partner across lane bit 2 (lane ^ 4) on DPP: row_shl:4 reads lane + 4,
// row_shr:4 lane - 4.
__device__ __forceinline__ float dpp_xor4(float v) {
    const float up = dpp_f<0x104>(v), dn = dpp_f<0x114>(v);
    return (threadIdx.x & 4) ? dn : up;
}

// Max over the wave, the same value in every lane: quads, half rows and rows
// on DPP (every pairing is exact for a max), then the 4 rows by readlane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Sum over aligned groups of N consecutive lanes (N <= 32) on DPP (a
// cross-row step for N = 32); the group's first lane holds the sum in a
// fixed order (other lanes may hold it in another).
template <uint32_t N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) v += dpp_f<0xB1>(v);
    if constexpr (N >= 4) v += dpp_f<0x4E>(v);
    if constexpr (N >= 8) v += dpp_xor4(v);
    if constexpr (N >= 16) v += dpp_f<0x128>(v);  // row_ror:8 (lane ^ 8 within a row)
    if constexpr (N >= 32) v += __shfl_xor(v, 16);
    return v;
}

// Sum over the wave in a fixed order (rows on DPP, then the 4 rows in order).
__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum<16>(v);
    return ((lane_f(v, 0) + lane_f(v, 16)) + lane_f(v, 32)) + lane_f(v, 48);
}

__device__ __forceinline__ float dot_tree8(float s) {
    const float t = s + dpp_f<0x104>(s);  // row_shl:4: l < 4 -> S_l + S_{l+4}
    const float u = t + dpp_f<0xB1>(t);   // quad_perm [1,0,3,2]: l=0 -> T0+T1, l=2 -> T2+T3
    return u + dpp_f<0x4E>(u);            // quad_perm [2,3,0,1]: l=0 -> (T0+T1)+(T2+T3)
}

template <uint32_t group>
__global__ __launch_bounds__(256) void k_attn_scores(const float* __restrict__ q, const float* __restrict__ kv,
                                                     const uint32_t* __restrict__ pos_p,
                                                     uint32_t head_stride, uint32_t n_heads, uint32_t max_seq,
                                                     float scale, float* __restrict__ scores,
                                                     float* __restrict__ part_max, uint32_t n_chunks) {
    const uint32_t S = *pos_p + 1u;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y;
    const uint32_t j0 = chunk * kChunk;
    if (j0 >= S) return;
    __shared__ float smax[4][kMaxGroup];
    // This workgroup's q rows and each wave's 16 K rows, staged in LDS with
    // coalesced 16-byte loads (the dot reads them in the reference's
    // stride-8 element order); K rows padded to kKs floats so that the
    // stride-8 reads of 8 keys fall in distinct banks.
    constexpr uint32_t kKs = kHd + 8;
    constexpr uint32_t kQPieces = group * kHd / 4;
    __shared__ float s_q[group * kHd];
    __shared__ float s_k[4][16][kKs];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 3, l = lane & 7;  // key slot g of the pass, reference lane l
    const float* kbase = kv + (size_t)kvh * head_stride;
    float4 kr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // piece pc of the wave's 16 rows: row pc/32, floats 4*(pc%32) ..; keys
        // past S read row j0 (in bounds) and are masked below
        const uint32_t pc = (uint32_t)(i * 64 + lane), k = pc >> 5, f = (pc & 31u) * 4u;
        const uint32_t j = j0 + (uint32_t)wave * 16u + k;
        kr[i] = *reinterpret_cast<const float4*>(kbase + (size_t)(j < S ? j : j0) * (2 * kHd) + f);
    }
    float4 qr = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (threadIdx.x < kQPieces) qr = *reinterpret_cast<const float4*>(q + (size_t)kvh * group * kHd + threadIdx.x * 4u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t pc = (uint32_t)(i * 64 + lane), k = pc >> 5, f = (pc & 31u) * 4u;
        *reinterpret_cast<float4*>(&s_k[wave][k][f]) = kr[i];
    }
    if (threadIdx.x < kQPieces) *reinterpret_cast<float4*>(&s_q[threadIdx.x * 4u]) = qr;
    __syncthreads();
    // q values this lane multiplies: q[h][32t + 8c + l]
    float qv[group][4][4];
#pragma unroll
    for (uint32_t h = 0; h < group; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) qv[h][c][t] = s_q[h * kHd + 32 * t + 8 * c + l];
    float mx[group];
#pragma unroll
    for (uint32_t h = 0; h < group; ++h) mx[h] = -INFINITY;
    // 64 keys per workgroup: each wave takes 16 in two passes of 8 (one key
    // per 8-lane group).
    float kk[2][4][4];
#pragma unroll
    for (int ps = 0; ps < 2; ++ps)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) kk[ps][c][t] = s_k[wave][ps * 8 + g][32 * t + 8 * c + l];
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
        const uint32_t j = j0 + (uint32_t)(wave * 16 + ps * 8 + g);
        const bool valid = j < S;
#pragma unroll
        for (uint32_t h = 0; h < group; ++h) {
            float a[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float acc = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) acc = fmaf(qv[h][c][t], kk[ps][c][t], acc);
                a[c] = acc;
            }
            const float sl = (a[0] + a[1]) + (a[2] + a[3]);
            const float d = dot_tree8(sl);
            const float sc = d * scale;
            if (valid && l == 0) scores[(size_t)(kvh * group + h) * max_seq + j] = sc;
            if (valid) mx[h] = fmaxf(mx[h], sc);
        }
    }
    // per-head max over the chunk: lanes l = 0 hold their keys' values; the
    // max is exact, so any combination order gives the same result.
#pragma unroll
    for (uint32_t h = 0; h < group; ++h) {
        const float m = wave_max((l == 0) ? mx[h] : -INFINITY);
        if (lane == 0) smax[wave][h] = m;
    }
    __syncthreads();
    if (threadIdx.x < group) {
        const uint32_t h = threadIdx.x;
        const float m = fmaxf(fmaxf(smax[0][h], smax[1][h]), fmaxf(smax[2][h], smax[3][h]));
        part_max[(size_t)(kvh * group + h) * n_chunks + chunk] = m;
    }
}

// Phase B over 256-key chunks, each split in 4 workgroups by 32-column
// slices of V (288 workgroups at context 2048, each reading 256 rows of 128
// bytes): the combine then sums at most 32 partials, one round of loads.
constexpr uint32_t kPvChunk = 256;
constexpr uint32_t kPvSlices = kHd / 32;

template <uint32_t group>
__global__ __launch_bounds__(256) void k_attn_pv(const float* __restrict__ scores, const float* __restrict__ kv,
                                                 const uint32_t* __restrict__ pos_p,
                                                 uint32_t head_stride, uint32_t n_heads, uint32_t max_seq,
                                                 const float* __restrict__ part_max, uint32_t n_chunks,
                                                 float* __restrict__ part_sum, float* __restrict__ o_part) {
    const uint32_t S = *pos_p + 1u;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, sl = blockIdx.z;
    const uint32_t j0 = chunk * kPvChunk;
    if (j0 >= S) return;
    const uint32_t nch = (S + kChunk - 1) / kChunk;  // score chunks holding part_max
    const uint32_t Sv = S >= 8 ? (S & ~7u) : 0u;     // polynomial exp below Sv, expf above
    constexpr uint32_t kThr = 32 / group;            // threads per output float4 in the final sum
    __shared__ __attribute__((aligned(16))) float e_s[group][kPvChunk];
    __shared__ float4 red[32][group][8];
    __shared__ float gmax[kMaxGroup];
    const uint32_t tid = threadIdx.x;
    const uint32_t r = tid >> 3, q = tid & 7;  // rows r, r+32, ..; float4 q of the 32-column slice
    // Loads that do not depend on the global max first: this thread's 8 V
    // pieces (rows past S read row S-1, in bounds; their e is 0) and the
    // chunk's scores.
    const float* vbase = kv + (size_t)kvh * head_stride + kHd + 32 * sl + 4 * q;
    float4 vv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t j = j0 + r + 32u * (uint32_t)k;
        vv[k] = *reinterpret_cast<const float4*>(vbase + (size_t)(j < S ? j : S - 1u) * (2 * kHd));
    }
    float scv[group];
    const uint32_t jt = j0 + tid;
#pragma unroll
    for (uint32_t h = 0; h < group; ++h)
        scv[h] = scores[(size_t)(kvh * group + h) * max_seq + (jt < S ? jt : S - 1u)];
    // Global max per head: one wave per head (lane-strided loads, then a
    // wave max); exact, so the order does not matter.
    const uint32_t wv = tid >> 6, ln = tid & 63;
    for (uint32_t hh = wv; hh < group; hh += 4) {
        const uint32_t h = kvh * group + hh;
        float m = -INFINITY;
        for (uint32_t c = ln; c < nch; c += 64) m = fmaxf(m, part_max[(size_t)h * n_chunks + c]);
        m = wave_max(m);
        if (ln == 0) gmax[hh] = m;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t h = 0; h < group; ++h) {
        float e = 0.0f;
        if (jt < S) {
            const float dd = scv[h] - gmax[h];
            e = (jt < Sv) ? exp_approx(dd) : expf(dd);
        }
        e_s[h][tid] = e;
    }
    __syncthreads();
    // The chunk's sums (slice 0): lane ln adds keys 4ln..4ln+3 in order, then
    // a fixed-order wave sum.
    if (sl == 0) {
        for (uint32_t hh = wv; hh < group; hh += 4) {
            const float4 e4 = *reinterpret_cast<const float4*>(&e_s[hh][4 * ln]);
            const float sum = wave_sum(((e4.x + e4.y) + e4.z) + e4.w);
            if (ln == 0) part_sum[(size_t)(kvh * group + hh) * n_chunks + chunk] = sum;
        }
    }
    // P.V over this thread's 8 rows for every head of the group.
    float4 acc[group];
#pragma unroll
    for (uint32_t h = 0; h < group; ++h) acc[h] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t jj = r + 32u * (uint32_t)k;
#pragma unroll
        for (uint32_t h = 0; h < group; ++h) {
            const float e = e_s[h][jj];
            acc[h].x = fmaf(e, vv[k].x, acc[h].x);
            acc[h].y = fmaf(e, vv[k].y, acc[h].y);
            acc[h].z = fmaf(e, vv[k].z, acc[h].z);
            acc[h].w = fmaf(e, vv[k].w, acc[h].w);
        }
    }
#pragma unroll
    for (uint32_t h = 0; h < group; ++h) red[r][h][q] = acc[h];
    __syncthreads();
    // Sum over the 32 row groups: output float4 (h, q) by kThr consecutive
    // threads, each over `group` row groups in order, then a lane-group sum.
    {
        const uint32_t o = tid / kThr, sub = tid % kThr;
        const uint32_t h = o >> 3, qq = o & 7u;
        float4 v = red[sub * group][h][qq];
#pragma unroll
        for (uint32_t i = 1; i < group; ++i) {
            const float4 w = red[sub * group + i][h][qq];
            v.x += w.x;
            v.y += w.y;
            v.z += w.z;
            v.w += w.w;
        }
        v.x = group_sum<kThr>(v.x);
        v.y = group_sum<kThr>(v.y);
        v.z = group_sum<kThr>(v.z);
        v.w = group_sum<kThr>(v.w);
        if (sub == 0)
            *reinterpret_cast<float4*>(o_part + ((size_t)chunk * n_heads + kvh * group + h) * kHd + 32 * sl + 4 * qq) = v;
    }
}

// o = (sum_c o_part[c]) * (1 / sum_c part_sum[c]) (for S < 8, the reference's
// scalar softmax divides: o = sum / total), then its digits for the Wo GEMV.
constexpr uint32_t kCombThreads = 64;  // more, smaller workgroups: the combine is one round of loads

__global__ __launch_bounds__(kCombThreads) void k_attn_combine(const float* __restrict__ o_part,
                                                      const float* __restrict__ part_sum,
                                                      const uint32_t* __restrict__ pos_p, uint32_t n_heads,
                                                      uint32_t n_chunks, float* __restrict__ o_out,
                                                      uint32_t pad, uint32_t* __restrict__ xd) {
    const uint32_t S = *pos_p + 1u;
    const uint32_t nch = (S + kPvChunk - 1) / kPvChunk;
    const uint32_t t = blockIdx.x * kCombThreads + threadIdx.x;  // element of o
    const uint32_t N = n_heads * kHd;
    const bool valid = t < N;
    float v = 0.0f;
    if (valid) {
        const uint32_t h = t / kHd;
        float total = 0.0f, acc = 0.0f;
        // Rounds of 32 chunks with every load of a round in flight together
        // (indices clamped in bounds, contributions past nch zeroed); the
        // sums stay sequential in chunk order.
        for (uint32_t c0 = 0; c0 < nch; c0 += 32) {
            float ps[32], op[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const uint32_t c = c0 + (uint32_t)u;
                const uint32_t cc = c < nch ? c : nch - 1u;
                ps[u] = part_sum[(size_t)h * n_chunks + cc];
                op[u] = o_part[(size_t)cc * N + t];
            }
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                if (c0 + (uint32_t)u < nch) {
                    total += ps[u];
                    acc += op[u];
                }
            }
        }
        if (S < 8) {
            v = acc / total;
        } else {
            const float inv = 1.0f / total;
            v = acc * inv;
        }
        if (o_out) o_out[t] = v;
    }
    prep_lane(v, t >> 5, valid, pad, xd);
}

template <uint32_t group>
static hipError_t run_attention(const AttnArgs& a, hipStream_t s) {
    const uint32_t n_chunks = (a.max_seq + kChunk - 1) / kChunk;
    const uint32_t head_stride = a.max_seq * 2 * kHd;
    dim3 grid(n_chunks, a.n_kv);
    hipLaunchKernelGGL(k_attn_scores<group>, grid, dim3(256), 0, s, a.q, a.kv_layer, a.pos, head_stride,
                       a.n_heads, a.max_seq, a.scale, a.scores, a.part_max, n_chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid_pv((a.max_seq + kPvChunk - 1) / kPvChunk, a.n_kv, kPvSlices);
    hipLaunchKernelGGL(k_attn_pv<group>, grid_pv, dim3(256), 0, s, a.scores, a.kv_layer, a.pos, head_stride,
                       a.n_heads, a.max_seq, a.part_max, n_chunks, a.part_sum, a.o_part);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t N = a.n_heads * kHd;
    hipLaunchKernelGGL(k_attn_combine, dim3((N + kCombThreads - 1) / kCombThreads), dim3(kCombThreads), 0, s,
                       a.o_part, a.part_sum, a.pos,
                       a.n_heads, n_chunks, a.o_out, xd_pad(N / 32), reinterpret_cast<uint32_t*>(a.xd_out));
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
    if (a.head_dim != kHd || a.n_kv == 0 || a.n_heads % a.n_kv != 0) return hipErrorInvalidValue;
    switch (a.n_heads / a.n_kv) {
        case 1: return run_attention<1>(a, s);
        case 2: return run_attention<2>(a, s);
        case 4: return run_attention<4>(a, s);
        case 8: return run_attention<8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

size_t attention_n_chunks(uint32_t max_seq) { return (max_seq + kChunk - 1) / kChunk; }

size_t attention_scratch_floats(uint32_t n_heads, uint32_t max_seq) {
    const uint32_t n_chunks = (max_seq + kChunk - 1) / kChunk;
    // scores + part_max + part_sum + o_part
    return (size_t)n_heads * max_seq + 2 * (size_t)n_heads * n_chunks + (size_t)n_chunks * n_heads * kHd;
}

// m = silu(g) * u (reference silu.c:75-82 then mul_fp32.c), then m's digits
// for the W_down GEMV.  N % 8 == 0 here (hidden_dim is a multiple of 32), so
// every element takes the polynomial path, as in the reference.
__global__ __launch_bounds__(256) void k_swiglu_prep(const float* __restrict__ g, const float* __restrict__ u,
                                                     uint32_t N, float* __restrict__ m_out, uint32_t pad,
                                                     uint32_t* __restrict__ xd) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    const bool valid = t < N;
    float v = 0.0f;
    if (valid) {
        const float sg = silu_approx(g[t]);
        v = sg * u[t];
        if (m_out) m_out[t] = v;
    }
    prep_lane(v, t >> 5, valid, pad, xd);
}

hipError_t launch_swiglu_prep(const float* g, const float* u, uint32_t N, float* m_out, uint4* xd, hipStream_t s) {
    if (N % 32 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_swiglu_prep, dim3((N + 255) / 256), dim3(256), 0, s, g, u, N, m_out, xd_pad(N / 32),
                       reinterpret_cast<uint32_t*>(xd));
    return hipGetLastError();
}

// x = embd[token] (reference model.c:1027-1068), token read from device
// memory; out-of-range tokens are clamped (the host validates the tokens it
// submits; a device-fed token is an argmax result, always < vocab).
__global__ __launch_bounds__(256) void k_embed(const float* __restrict__ embd, const uint32_t* __restrict__ tok,
                                               uint32_t vocab, uint32_t dim, float* __restrict__ x) {
    uint32_t t = *tok;
    t = t < vocab ? t : vocab - 1;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < dim; i += gridDim.x * 256)
        x[i] = embd[(size_t)t * dim + i];
}

hipError_t launch_embed(const float* embd, const uint32_t* tok, uint32_t vocab, uint32_t dim, float* x,
                        hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3((dim + 255) / 256), dim3(256), 0, s, embd, tok, vocab, dim, x);
    return hipGetLastError();
}

}  // namespace qh
