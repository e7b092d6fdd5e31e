// api_sample.cpp -- q_sample_token (reference src/main.c:852-992) on the GPU.
//
// Validation order, return codes, the arena allocations (same sizes, same
// order, so the arena ends where the reference's does and runs out where
// it does), the thread-local xorshift64* stream and the draw
// r = (u32 >> 8) / 2^24 are the reference's; the arithmetic runs on the
// device (k_sample.hip).  Two rules where the reference's behaviour is not
// defined by its inputs:
//   * equal probabilities at a top-k / top-p cut keep the lower indices
//     (the reference's choice follows its quickselect/quicksort internals);
//   * with neither top-k nor top-p, every token is valid (the reference
//     reads a mask that nothing wrote).
// Without an arena the reference's softmax path depends on the alignment
// malloc returns; this build takes the aligned (vector) path, the one the
// arena gives.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "qh_kernels.hpp"
#include "qh_runtime.hpp"
#include "qh_sample.hpp"

namespace qh {
namespace {

thread_local uint64_t g_rng_state = 123456789ULL;  // reference main.c:949

// xorshift64* step and the [0, 1) draw of reference main.c:965-968.
float next_uniform() {
    uint64_t x = g_rng_state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    g_rng_state = x;
    const uint32_t u = (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
    return (float)(u >> 8) / 16777216.0f;
}

// The reference's arena-backed prob_array_t: the struct, then indices and
// probabilities (main.c:205-237).  False when any allocation fails.
bool arena_prob_array(q_context* ctx, uint32_t V) {
    if (!q_arena_alloc(ctx, 24)) return false;  // sizeof(prob_array_t) on LP64
    if (!q_arena_alloc(ctx, Q_ALIGN_SIZE((size_t)V * sizeof(uint32_t)))) return false;
    if (!q_arena_alloc(ctx, Q_ALIGN_SIZE((size_t)V * sizeof(float)))) return false;
    return true;
}

}  // namespace

float sample_draw() { return next_uniform(); }

}  // namespace qh

using namespace qh;

extern "C" {

q_error_code q_sample_token(const float* __restrict__ logits, uint32_t vocab_size, float temperature, uint32_t top_k,
                            float top_p, uint32_t* __restrict__ token_id_out, q_context* __restrict__ ctx) {
    if (!logits || !token_id_out) return Q_ERR_INVALID_ARG;
    if (vocab_size == 0) return Q_ERR_INVALID_SIZE;
    if (!(temperature >= 0.0f) || !std::isfinite(temperature)) return Q_ERR_INVALID_ARG;
    const uint32_t V = vocab_size;
    Device* d;
    if (temperature < 1e-6f) {  // greedy: first index of the maximum
        QH_TRY_CODE(device(&d));
        std::lock_guard<std::mutex> lk(d->mu);
        void* buf;
        QH_TRY_CODE(stage(d, 1, (size_t)V * 4 + 256, &buf));
        float* dl = static_cast<float*>(buf);
        uint32_t* di = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(buf) + (((size_t)V * 4 + 255) & ~(size_t)255));
        QH_TRY_CODE(h2d_pinned(d, dl, logits, (size_t)V * 4));
        QH_TRY(launch_argmax_ws(dl, V, di, nullptr, nullptr, nullptr, 0, d->reduce_ws, d->stream));
        QH_TRY(hipMemcpyAsync(token_id_out, di, 4, hipMemcpyDeviceToHost, d->stream));
        QH_TRY(hipStreamSynchronize(d->stream));
        return Q_OK;
    }
    // The reference's allocations, in its order (main.c:891-899, 431-470,
    // 720-760, 525-549).
    const bool use_arena = ctx && ctx->scratch_buffer;
    SampleParams sp;
    if (use_arena) {
        void* probs = q_arena_alloc(ctx, Q_ALIGN_SIZE((size_t)V * sizeof(float)));
        void* mask = q_arena_alloc(ctx, Q_ALIGN_SIZE((size_t)V * sizeof(bool)));
        if (!probs || !mask) return Q_ERR_ARENA_OOM;
        if (top_k > 0 && top_k < V && !arena_prob_array(ctx, V)) return Q_ERR_ARENA_OOM;
        if (top_p > 0.0f && top_p < 1.0f) {
            if (!arena_prob_array(ctx, V)) return Q_ERR_ARENA_OOM;
            if (!q_arena_alloc(ctx, Q_ALIGN_SIZE((size_t)V * sizeof(float)))) sp.nucleus_all = true;
        }
    }
    sp.vocab = V;
    sp.temperature = temperature;
    sp.inv_temperature = 1.0f / temperature;
    // 8-wide multiply by 1/T when the logits are 32-byte aligned
    // (main.c:338-365); the probability buffer is taken as aligned.
    sp.n_mul = (V >= 8 && (reinterpret_cast<uintptr_t>(logits) % 32) == 0) ? (V & ~7u) : 0u;
    sp.top_k = top_k;
    sp.top_p = top_p;
    QH_TRY_CODE(device(&d));
    sp.r = next_uniform();
    std::lock_guard<std::mutex> lk(d->mu);
    const size_t lb = ((size_t)V * 4 + 255) & ~(size_t)255;
    const size_t wb = sample_workspace_bytes(V);
    if (wb == 0) return fail(hipErrorInvalidValue, "q_sample_token: workspace size");
    void* buf;
    QH_TRY_CODE(stage(d, 1, lb + 256 + wb, &buf));
    uint8_t* B = static_cast<uint8_t*>(buf);
    float* dl = reinterpret_cast<float*>(B);
    uint32_t* dt = reinterpret_cast<uint32_t*>(B + lb);
    QH_TRY_CODE(h2d_pinned(d, dl, logits, (size_t)V * 4));
    QH_TRY(launch_sample(dl, sp, B + lb + 256, dt, d->stream));
    QH_TRY(hipMemcpyAsync(token_id_out, dt, 4, hipMemcpyDeviceToHost, d->stream));
    QH_TRY(hipStreamSynchronize(d->stream));
    return Q_OK;
}

// The calling thread's sampling RNG state (no reference counterpart: the
// reference keeps it private; these make a run reproducible).
void qh_sample_set_state(uint64_t state) { g_rng_state = state; }
uint64_t qh_sample_get_state(void) { return g_rng_state; }

}  // extern "C"
