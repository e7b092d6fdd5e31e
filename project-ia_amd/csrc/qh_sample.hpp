// qh_sample.hpp -- on-device token sampling (k_sample.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qh {

struct SampleParams {
    uint32_t vocab = 0;
    float temperature = 1.0f;      // > 0 (temperature 0 is the greedy argmax, not this path)
    float inv_temperature = 1.0f;  // 1.0f / temperature (the reference's vector divide)
    uint32_t n_mul = 0;            // logits [0, n_mul) scaled by inv_temperature, the rest divided
    uint32_t top_k = 0;            // 0: off
    float top_p = 0.0f;            // <= 0: off
    bool nucleus_all = false;      // top-p keeps every token (the reference's prefix-sum buffer failed)
    float r = 0.0f;                // uniform draw in [0, 1)
};

// The calling thread's next uniform draw in [0, 1) (the reference's
// xorshift64* stream, advanced once).
float sample_draw();

// After a sampled generation step: hist[*hist_n] = *tok (if it fits),
// ++*hist_n, ++*pos.
hipError_t launch_token_feedback(const uint32_t* tok, uint32_t* pos, uint32_t* hist, uint32_t* hist_n,
                                 uint32_t hist_cap, hipStream_t s);

// Device workspace bytes launch_sample needs for a vocabulary of V.
size_t sample_workspace_bytes(uint32_t V);
// Samples one token from device logits[V] into *token (device memory).
hipError_t launch_sample(const float* logits, const SampleParams& sp, void* ws, uint32_t* token, hipStream_t s);

}  // namespace qh
