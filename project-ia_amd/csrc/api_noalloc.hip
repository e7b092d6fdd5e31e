// api_noalloc.hip -- the allocation-free form of the LM-head entry point
// (qh_gemv_q4_f32_softmax_argmax_noalloc).  Its scratch (the softmax's slice
// partials and the GEMV's argmax partials) is a file-scope device array, one
// per GPU for the life of the process, so a call allocates nothing.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "qh_kernels.hpp"
#include "qh_runtime.hpp"

namespace qh {

// Largest need: 1024 softmax slices (4*1024 + 8 floats, 256-byte aligned)
// plus 1024 argmax partials (value, index): 24,832 bytes, for every M.
constexpr size_t kScratchBytes = 32768;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` on each GPU, taken once per device with that
// device current.  In host code the array's name is only a stand-in for the
// symbol; every host use (kernel arguments) goes through these addresses.
constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

q_error_code noalloc_scratch_init(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return fail(hipErrorInvalidDevice, "qh noalloc scratch: device index");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[dev].load(std::memory_order_relaxed)) return Q_OK;
    void* p = nullptr;
    QH_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(hipErrorInvalidSymbol, "qh noalloc scratch: no device address");
    g_scratch[dev].store(p, std::memory_order_release);
    return Q_OK;
}

// The address on the current device: taken at the library's device
// initialization for its device, here (once) for any other.
static q_error_code scratch_address(void** out) {
    int dev = 0;
    QH_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(hipErrorInvalidDevice, "qh noalloc scratch: device index");
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        QH_TRY_CODE(noalloc_scratch_init(dev));
        p = g_scratch[dev].load(std::memory_order_acquire);
    }
    *out = p;
    return Q_OK;
}

}  // namespace qh

using namespace qh;

extern "C" q_error_code qh_gemv_q4_f32_softmax_argmax_noalloc(const q_tensor* W, const float* x, float* logits,
                                                              float* probs, uint32_t* index_out, qh_stream s) {
    QH_TRY_CODE(validate_gemv_softmax(W, x, logits, probs, index_out, false, nullptr));
    if (W->ne[1] / 32 > kGemvF32MaxBlk)
        return fail_code(Q_ERR_INVALID_SIZE,
                         "qh_gemv_q4_f32_softmax_argmax_noalloc: N above 16384 would need a digit workspace");
    if (gemv_softmax_ws_bytes(W->ne[0]) > kScratchBytes)
        return fail_code(Q_ERR_INVALID_SIZE, "qh_gemv_q4_f32_softmax_argmax_noalloc: partials exceed the 32 KB scratch");
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY_CODE(check_gemv_softmax_memory(W, x, logits, probs, index_out, nullptr));
    void* ws = nullptr;
    QH_TRY_CODE(scratch_address(&ws));
    return gemv_softmax_argmax_run(W, x, logits, probs, index_out, ws, false, (hipStream_t)s);
}
