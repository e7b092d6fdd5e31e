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
// found first.  Three phases, keys split in chunks of kChunk:
//   A  scores + per-chunk max           grid (chunks, kv heads)
//   B  e_j, per-chunk sums and P.V sums  grid (chunks, kv heads)
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
        float m = (l == 0) ? mx[h] : -INFINITY;
#pragma unroll
        for (int off = 8; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (lane == 0) smax[wave][h] = m;
    }
    __syncthreads();
    if (threadIdx.x < group) {
        const uint32_t h = threadIdx.x;
        const float m = fmaxf(fmaxf(smax[0][h], smax[1][h]), fmaxf(smax[2][h], smax[3][h]));
        part_max[(size_t)(kvh * group + h) * n_chunks + chunk] = m;
    }
}

template <uint32_t group>
__global__ __launch_bounds__(256) void k_attn_pv(const float* __restrict__ scores, const float* __restrict__ kv,
                                                 const uint32_t* __restrict__ pos_p,
                                                 uint32_t head_stride, uint32_t n_heads, uint32_t max_seq,
                                                 const float* __restrict__ part_max, uint32_t n_chunks,
                                                 float* __restrict__ part_sum, float* __restrict__ o_part) {
    const uint32_t S = *pos_p + 1u;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y;
    const uint32_t j0 = chunk * kChunk;
    if (j0 >= S) return;
    const uint32_t nch = (S + kChunk - 1) / kChunk;
    const uint32_t Sv = S >= 8 ? (S & ~7u) : 0u;  // polynomial exp below Sv, expf above
    __shared__ float e_s[kMaxGroup][kChunk];
    __shared__ float o_s[kMaxGroup][kHd];
    __shared__ float gmax[kMaxGroup];
    const uint32_t tid = threadIdx.x;
    // Loads that do not depend on the global max are issued first: this
    // chunk's V rows (thread (hf, d): keys hf*32 .. hf*32+31, element d) and
    // its scores.  Keys past S read a clamped, in-bounds row and are zeroed.
    const uint32_t d = tid % kHd, hf = tid / kHd;
    const float* vbase = kv + (size_t)kvh * head_stride + kHd;
    float vv[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) {
        const uint32_t j = j0 + hf * 32 + (uint32_t)u;
        const float v = vbase[(size_t)(j < S ? j : S - 1u) * (2 * kHd) + d];
        vv[u] = (j < S) ? v : 0.0f;
    }
    constexpr uint32_t kPer = (group * kChunk + 255) / 256;
    float scv[kPer];
#pragma unroll
    for (uint32_t r = 0; r < kPer; ++r) {
        const uint32_t i = tid + 256 * r;
        const uint32_t h = i / kChunk, jj = i % kChunk, j = j0 + jj;
        const bool ok = i < group * kChunk && j < S;
        const uint32_t hc = h < group ? h : 0u;
        const float sv = scores[(size_t)(kvh * group + hc) * max_seq + (j < S ? j : S - 1u)];
        scv[r] = ok ? sv : 0.0f;
    }
    // Global max per head: one wave per head (lane-strided loads, then a
    // butterfly max); exact, so the order does not matter.
    {
        const uint32_t wv = tid >> 6, ln = tid & 63;
        for (uint32_t hh = wv; hh < group; hh += 4) {
            const uint32_t h = kvh * group + hh;
            float m = -INFINITY;
            for (uint32_t c = ln; c < nch; c += 64) m = fmaxf(m, part_max[(size_t)h * n_chunks + c]);
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
            if (ln == 0) gmax[hh] = m;
        }
    }
    __syncthreads();
    // e_j for the chunk's keys and all group heads.
#pragma unroll
    for (uint32_t r = 0; r < kPer; ++r) {
        const uint32_t i = tid + 256 * r;
        if (i < group * kChunk) {
            const uint32_t h = i / kChunk, jj = i % kChunk, j = j0 + jj;
            float e = 0.0f;
            if (j < S) {
                const float dd = scv[r] - gmax[h];
                e = (j < Sv) ? exp_approx(dd) : expf(dd);
            }
            e_s[h][jj] = e;
        }
    }
    __syncthreads();
    if (tid < group) {
        float sum = 0.0f;
        for (int jj = 0; jj < kChunk; ++jj) sum += e_s[tid][jj];
        part_sum[(size_t)(kvh * group + tid) * n_chunks + chunk] = sum;
    }
    // P.V partials: thread (half, d) over its 32 keys, all group heads.
    float acc[group];
#pragma unroll
    for (uint32_t h = 0; h < group; ++h) acc[h] = 0.0f;
#pragma unroll
    for (int u = 0; u < 32; ++u) {
        const int jj = (int)hf * 32 + u;
#pragma unroll
        for (uint32_t h = 0; h < group; ++h) acc[h] = fmaf(e_s[h][jj], vv[u], acc[h]);
    }
    if (hf == 1)
#pragma unroll
        for (uint32_t h = 0; h < group; ++h) o_s[h][d] = acc[h];
    __syncthreads();
    if (hf == 0)
#pragma unroll
        for (uint32_t h = 0; h < group; ++h)
            o_part[((size_t)chunk * n_heads + kvh * group + h) * kHd + d] = acc[h] + o_s[h][d];
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
    const uint32_t nch = (S + kChunk - 1) / kChunk;
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
    hipLaunchKernelGGL(k_attn_pv<group>, grid, dim3(256), 0, s, a.scores, a.kv_layer, a.pos, head_stride,
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
