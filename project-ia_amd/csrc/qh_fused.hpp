// qh_fused.hpp -- launchers of the decode step's fused GEMVs (k_fused.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qh_kernels.hpp"

namespace qh {

struct FusedArgs {
    // Q4_0 matrices: w[0] (RESID: Wo), or w[0], w[1] = W_gate, W_up (SWIGLU).
    const uint8_t* w[2] = {nullptr, nullptr};
    uint32_t M[2] = {0, 0};
    uint32_t nseg = 0;
    // Input: digit planes (uint4 [7][pad]) of N = 32*nblk elements and, for
    // SWIGLU (an RMSNorm output), the per-block sums of squares of the
    // un-normalized vector plus eps.
    uint32_t nblk = 0;
    uint32_t pad = 0;
    const uint4* xd = nullptr;
    const float* in_part = nullptr;
    float eps = 0.0f;
    // RESID: y[0] = res + W.x; digits of y[0]*wnorm go to xd_out, per-block
    // sums of squares of y[0] to out_part.  SWIGLU: digits of silu(g)*u.
    float* y[1] = {nullptr};
    const float* res = nullptr;
    const float* wnorm = nullptr;
    uint4* xd_out = nullptr;
    uint32_t pad_out = 0;
    float* out_part = nullptr;
};

// Whether the fused kernels handle an input of nblk blocks (<= 128).
bool fused_supported(uint32_t nblk);
// y = res + W.x, and the next RMSNorm's input digits and block sums.
hipError_t launch_fused_resid(FusedArgs a, hipStream_t s);
// W_gate (w[0]) and W_up (w[1]) of an RMSNorm'd input; digits of silu(g)*u.
hipError_t launch_fused_swiglu(FusedArgs a, hipStream_t s);

}  // namespace qh
