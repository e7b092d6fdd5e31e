// qh_prefill.hpp -- launchers of the batched-prefill kernels (k_prefill.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qh {

// X[t] = embd[tok[t]] for t < T (tok: device, every entry < vocab).
hipError_t launch_embed_rows(const float* embd, const uint32_t* tok, uint32_t T, uint32_t dim, float* X,
                             hipStream_t s);

// RoPE of the Q rows in place and of the K rows into the KV cache, V rows
// copied to the cache: token t sits at position pos0 + t.  Q [T][n_heads*128],
// K and V [T][n_kv*128]; kv_layer is one layer's [n_kv][max_seq][K|V][128]
// cache; cos/sin tables [max_seq][128].  With part set, the Q|K|V rows are
// the Q|K|V GEMM's deferred split-K partials ([split][T][q | k | v], pmeta
// its per-token scales; K and V unused), reduced here in the reduction's
// own order, and Q is written.
hipError_t launch_rope_kv_rows(float* Q, const float* K, const float* V, const float* cos_tab,
                               const float* sin_tab, uint32_t pos0, uint32_t T, uint32_t n_heads, uint32_t n_kv,
                               uint32_t max_seq, float* kv_layer, hipStream_t s, const float* part = nullptr,
                               uint32_t split = 0, const float2* pmeta = nullptr);

// Causal attention of T queries at positions pos0 .. pos0+T-1 over the
// cache (query t attends keys 0 .. pos0+t, all already in the cache), the
// decode step's arithmetic per query: O [T][n_heads*128].
struct PrefillAttnArgs {
    const float* q;         // [T][n_heads*128], RoPE applied
    const float* kv;        // this layer's cache [n_kv][max_seq][2][128]
    float* o;               // [T][n_heads*128]
    uint32_t T, pos0, n_heads, n_kv, max_seq;
    float scale;            // 1/sqrtf(head_dim)
    void* khl;              // scratch, prefill_khl_bytes(n_kv, max_seq): the keys as
                            // scaled fp16 hi/lo rows and their exponents
};
// Bytes of PrefillAttnArgs::khl for a cache of n_kv heads x max_seq rows.
size_t prefill_khl_bytes(uint32_t n_kv, uint32_t max_seq);
hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t s);

}  // namespace qh
