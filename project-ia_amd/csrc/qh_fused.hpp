// qh_fused.hpp -- launchers of the decode step's fused GEMVs (k_fused.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qh_kernels.hpp"

namespace qh {

struct FusedArgs {
    // Q4_0 matrices (segments) sharing the input; rows are tiled in 32-row
    // output blocks (tile_end: cumulative tile counts, filled by the launcher).
    const uint8_t* w[3] = {nullptr, nullptr, nullptr};
    uint32_t M[3] = {0, 0, 0};
    uint32_t tile_end[3] = {0, 0, 0};
    uint32_t nseg = 0;
    // Input: digit planes (uint4 [7][pad]) of N = 32*nblk elements and, for
    // the consumers of an RMSNorm output, the per-block sums of squares of
    // the un-normalized vector plus eps.
    uint32_t nblk = 0;
    uint32_t pad = 0;
    const uint4* xd = nullptr;
    const float* in_part = nullptr;
    float eps = 0.0f;
    // Outputs.  QKV: y[i] is segment i's destination; with hd[i] > 0 row r
    // goes to y[i] + pos*pos_stride[i] + (r/hd)*head_stride[i] + r%hd, RoPE'd
    // when bit i of rope_mask is set.  LOGITS / RESID: y[0] [M].
    float* y[3] = {nullptr, nullptr, nullptr};
    uint32_t hd[3] = {0, 0, 0};
    uint32_t head_stride[3] = {0, 0, 0};
    uint32_t pos_stride[3] = {0, 0, 0};
    uint32_t rope_mask = 0;
    const uint32_t* pos = nullptr;
    const float* cos_tab = nullptr;
    const float* sin_tab = nullptr;
    // RESID: y[0] = res + W.x; digits of y[0]*wnorm go to xd_out, per-block
    // sums of squares of y[0] to out_part.  SWIGLU: digits of silu(g)*u.
    const float* res = nullptr;
    const float* wnorm = nullptr;
    uint4* xd_out = nullptr;
    uint32_t pad_out = 0;
    float* out_part = nullptr;
};

// Whether the fused kernels handle an input of nblk blocks.
bool fused_supported(uint32_t nblk);
// Q|K|V (up to 3 segments) of an RMSNorm'd input, RoPE and cache stores.
hipError_t launch_fused_qkv(FusedArgs a, hipStream_t s);
// y = res + W.x, and the next RMSNorm's input digits and block sums.
hipError_t launch_fused_resid(FusedArgs a, hipStream_t s);
// W_gate (w[0]) and W_up (w[1]) of an RMSNorm'd input; digits of silu(g)*u.
hipError_t launch_fused_swiglu(FusedArgs a, hipStream_t s);
// Logits of an RMSNorm'd input.
hipError_t launch_fused_logits(FusedArgs a, hipStream_t s);
// Embedding row of *tok into x, plus its RMSNorm input digits and block sums.
hipError_t launch_embed_prep(const float* embd, const uint32_t* tok, uint32_t vocab, uint32_t dim,
                             const float* wnorm, float* x, uint4* xd, float* part, hipStream_t s);

}  // namespace qh
