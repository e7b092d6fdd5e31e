// qh_runtime.hpp -- internal runtime of libqorus_hip.so: HIP error mapping,
// per-process device state (library stream, grow-only staging buffers) and
// the side table that attaches HBM state to a q_context without changing
// the q_context layout.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

#include "qorus.h"
#include "qorus_hip.h"

namespace qh {

// Records the HIP error text for qh_last_error() and maps it to a q_error_code.
q_error_code fail(hipError_t e, const char* what);
// Records `what` for qh_last_error() and returns code.
q_error_code fail_code(q_error_code code, const char* what);

#define QH_TRY(expr)                                        \
    do {                                                    \
        hipError_t qh_e_ = (expr);                          \
        if (qh_e_ != hipSuccess) return ::qh::fail(qh_e_, #expr); \
    } while (0)

#define QH_TRY_CODE(expr)                   \
    do {                                    \
        q_error_code qh_c_ = (expr);        \
        if (qh_c_ != Q_OK) return qh_c_;    \
    } while (0)

// Process-wide device state, created on first use.  Every HIP resource the
// library owns (stream, staging buffers) lives here; the op entry points of
// qorus.h run on `stream` and synchronize before returning.
struct Device {
    int id = -1;
    hipStream_t stream = nullptr;
    std::mutex mu;  // serializes the synchronous host-pointer entry points
    // Grow-only device staging used by the host-pointer entry points.
    void* stage[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t stage_bytes[4] = {0, 0, 0, 0};
    void* host_stage = nullptr;  // pinned host bounce buffer (hipHostMalloc)
    size_t host_stage_bytes = 0;
    // Partials of the multi-workgroup softmax/argmax used by the entry points
    // that take no workspace (allocated once at initialization).
    float* reduce_ws = nullptr;
    // Digit workspace of the GEMV entry points called without one (inputs
    // up to kLibGemvMaxN wide; allocated once at initialization).
    void* gemv_ws = nullptr;
};

constexpr size_t kReduceWsBytes = 65536;
constexpr uint32_t kLibGemvMaxN = 1u << 20;

// The no-allocation LM-head entry point's scratch address on device `dev`
// (taken once, with that device current; api_noalloc.hip).
q_error_code noalloc_scratch_init(int dev);

// Returns Q_OK and the initialized device, or an error if no GPU is usable.
q_error_code device(Device** out);

// Ensures staging slot `slot` holds at least `bytes`; returns its address.
q_error_code stage(Device* d, int slot, size_t bytes, void** out);
// Host -> device copy of `bytes` from pageable host memory through the
// device's pinned bounce buffer (a host memcpy, then one DMA on d->stream).
// The caller holds d->mu and synchronizes d->stream before the next use.
q_error_code h2d_pinned(Device* d, void* dst, const void* src, size_t bytes);

// HBM mirror of a q_context (side table keyed by the context address).
struct CtxState {
    q_context* ctx = nullptr;
    uint8_t* dev_weights = nullptr;  // HBM copy of the mapped .qorus file
    size_t weights_size = 0;
    uint8_t* dev_arena = nullptr;    // decode-step scratch (allocated by llama_build_graph)
    size_t dev_arena_size = 0;
    void* plan = nullptr;            // ModelPlan* (model.cpp)
};

CtxState* ctx_state(const q_context* ctx, bool create);
void ctx_state_erase(const q_context* ctx);

// If [p, p+bytes) lies inside the host mapping of a registered context whose
// weights are HBM-resident, returns the device address of p; else nullptr.
const void* resident_alias(const void* p, size_t bytes);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// GEMV argument checks of reference src/ops/avx2/matmul.c:104-197 plus the
// device-side ones (api_q4.cpp), shared by every GEMV entry point.
q_error_code validate_gemv(const q_tensor* W, const float* x, const float* y);

// LM head + softmax + greedy argmax (qh_gemv_q4_f32_softmax_argmax): the
// argument checks, the workspace size for M logits, and the launches on st
// with that workspace.  Inputs wider than the in-kernel digit conversion
// need a digit workspace, taken from the library's own allocation only when
// may_allocate (else the call fails).
size_t gemv_softmax_ws_bytes(uint32_t M);
// need_ws: a NULL workspace is refused with the other NULL arguments.
q_error_code validate_gemv_softmax(const q_tensor* W, const float* x, const float* logits, const float* probs,
                                   const uint32_t* index_out, bool need_ws, const void* workspace);
// After validation: every operand (and a non-NULL workspace) is device
// memory of the extent the launches touch, else Q_ERR_INVALID_ARG.
q_error_code check_gemv_softmax_memory(const q_tensor* W, const float* x, const float* logits, const float* probs,
                                       const uint32_t* index_out, const void* workspace);
q_error_code gemv_softmax_argmax_run(const q_tensor* W, const float* x, float* logits, float* probs,
                                     uint32_t* index_out, void* workspace, bool may_allocate, hipStream_t st);

// True when [p, p + bytes) lies inside one device-memory allocation known to
// the HIP runtime (hipMalloc, a caching allocator's block, ...).  Host
// pointers, unmapped addresses and ranges that run past their allocation
// give false, so an entry point can return an error code instead of
// launching a kernel on them.
bool device_range(const void* p, size_t bytes);

}  // namespace qh
