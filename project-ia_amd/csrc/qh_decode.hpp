// qh_decode.hpp -- launchers of the decode-step kernels (k_decode.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qh_kernels.hpp"

namespace qh {

struct AttnArgs {
    const float* q;        // [n_heads][head_dim], RoPE applied
    const float* kv_layer; // this layer's cache [n_kv][max_seq][2][head_dim]
    const uint32_t* pos;   // device: attend keys 0..*pos
    uint32_t n_heads, n_kv, head_dim, max_seq;
    float scale;           // 1/sqrtf(head_dim), computed on the host
    float* scores;         // scratch [n_heads][max_seq]
    float* part_max;       // scratch [n_heads][n_chunks]
    float* part_sum;       // scratch [n_heads][n_chunks]
    float* o_part;         // scratch [n_chunks][n_heads*head_dim]
    float* o_out;          // optional [n_heads*head_dim] attention output
    uint4* xd_out;         // digit planes of the output (Wo GEMV input)
};

hipError_t launch_attention(const AttnArgs& a, hipStream_t s);
// Floats of scratch launch_attention needs (scores + partials).
size_t attention_scratch_floats(uint32_t n_heads, uint32_t max_seq);
size_t attention_n_chunks(uint32_t max_seq);

hipError_t launch_swiglu_prep(const float* g, const float* u, uint32_t N, float* m_out, uint4* xd, hipStream_t s);
hipError_t launch_embed(const float* embd, const uint32_t* tok, uint32_t vocab, uint32_t dim, float* x,
                        hipStream_t s);

}  // namespace qh
