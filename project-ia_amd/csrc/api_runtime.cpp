// api_runtime.cpp -- device state, error reporting, the q_context side
// table, and the qh_* plumbing entry points of qorus_hip.h.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "qh_kernels.hpp"
#include "qh_runtime.hpp"

namespace qh {

static thread_local std::string g_last_error;
static std::mutex g_init_mu;
static Device* g_dev = nullptr;
static char g_arch[64] = "";

q_error_code fail(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory || e == hipErrorNoDevice || e == hipErrorInvalidDevice)
        return Q_ERR_ALLOC_FAILED;
    return Q_ERR_INVALID_ARG;
}

q_error_code fail_code(q_error_code code, const char* what) {
    g_last_error = what;
    return code;
}

q_error_code device(Device** out) {
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (!g_dev) {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n <= 0) {
            g_last_error = "no HIP device visible";
            return Q_ERR_ALLOC_FAILED;
        }
        int id = 0;
        QH_TRY(hipGetDevice(&id));
        hipDeviceProp_t prop;
        QH_TRY(hipGetDeviceProperties(&prop, id));
        std::snprintf(g_arch, sizeof(g_arch), "%s", prop.gcnArchName);
        Device* d = new Device();
        d->id = id;
        QH_TRY(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
        QH_TRY(hipMalloc(reinterpret_cast<void**>(&d->reduce_ws), kReduceWsBytes));
        QH_TRY(hipMalloc(&d->gemv_ws, xd_bytes(kLibGemvMaxN / 32)));
        QH_TRY_CODE(noalloc_scratch_init(id));
        g_dev = d;
    }
    *out = g_dev;
    return Q_OK;
}

q_error_code stage(Device* d, int slot, size_t bytes, void** out) {
    if (bytes == 0) bytes = 256;
    if (d->stage_bytes[slot] < bytes) {
        if (d->stage[slot]) {
            QH_TRY(hipStreamSynchronize(d->stream));
            QH_TRY(hipFree(d->stage[slot]));
            d->stage[slot] = nullptr;
            d->stage_bytes[slot] = 0;
        }
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        QH_TRY(hipMalloc(&d->stage[slot], want));
        d->stage_bytes[slot] = want;
    }
    *out = d->stage[slot];
    return Q_OK;
}

q_error_code h2d_pinned(Device* d, void* dst, const void* src, size_t bytes) {
    if (d->host_stage_bytes < bytes) {
        if (d->host_stage) {
            QH_TRY(hipStreamSynchronize(d->stream));
            QH_TRY(hipHostFree(d->host_stage));
            d->host_stage = nullptr;
            d->host_stage_bytes = 0;
        }
        const size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        QH_TRY(hipHostMalloc(&d->host_stage, want, hipHostMallocDefault));
        d->host_stage_bytes = want;
    }
    std::memcpy(d->host_stage, src, bytes);
    QH_TRY(hipMemcpyAsync(dst, d->host_stage, bytes, hipMemcpyHostToDevice, d->stream));
    return Q_OK;
}

// ---- q_context side table ----
static std::mutex g_ctx_mu;
static std::map<const q_context*, CtxState*> g_ctx;

CtxState* ctx_state(const q_context* ctx, bool create) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    auto it = g_ctx.find(ctx);
    if (it != g_ctx.end()) return it->second;
    if (!create) return nullptr;
    CtxState* st = new CtxState();
    st->ctx = const_cast<q_context*>(ctx);
    g_ctx[ctx] = st;
    return st;
}

void ctx_state_erase(const q_context* ctx) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    auto it = g_ctx.find(ctx);
    if (it == g_ctx.end()) return;
    delete it->second;
    g_ctx.erase(it);
}

const void* resident_alias(const void* p, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    for (auto& kv : g_ctx) {
        const CtxState* st = kv.second;
        const q_context* c = st->ctx;
        if (!st->dev_weights || !c->weights_mmap) continue;
        const uintptr_t b = reinterpret_cast<uintptr_t>(c->weights_mmap);
        if (a >= b && a + bytes <= b + c->weights_size && a + bytes >= a)
            return st->dev_weights + (a - b);
    }
    return nullptr;
}

bool device_range(const void* p, size_t bytes) {
    if (!p) return false;
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();  // an unknown address is an answer, not an error to keep
        return false;
    }
    if (at.type != hipMemoryTypeDevice && !at.isManaged) return false;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(base);
    return a >= b && bytes <= size && a - b <= size - bytes;
}

}  // namespace qh

using namespace qh;

extern "C" {

int qh_available(void) {
    Device* d = nullptr;
    return device(&d) == Q_OK ? 1 : 0;
}

const char* qh_last_error(void) { return g_last_error.c_str(); }

const char* qh_arch_name(void) {
    Device* d = nullptr;
    if (device(&d) != Q_OK) return "";
    return g_arch;
}

q_error_code qh_malloc(void** ptr, size_t bytes) {
    if (!ptr) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    QH_TRY(hipMalloc(ptr, bytes ? bytes : 1));
    return Q_OK;
}

q_error_code qh_free(void* ptr) {
    if (!ptr) return Q_OK;
    QH_TRY(hipFree(ptr));
    return Q_OK;
}

q_error_code qh_memcpy_htod(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return Q_OK;
    if (!dst || !src) return Q_ERR_INVALID_ARG;
    QH_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return Q_OK;
}

q_error_code qh_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return Q_OK;
    if (!dst || !src) return Q_ERR_INVALID_ARG;
    QH_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return Q_OK;
}

q_error_code qh_memcpy_dtod(void* dst, const void* src, size_t bytes, qh_stream s) {
    if (bytes == 0) return Q_OK;
    if (!dst || !src) return Q_ERR_INVALID_ARG;
    QH_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_memset(void* dst, int value, size_t bytes, qh_stream s) {
    if (bytes == 0) return Q_OK;
    if (!dst) return Q_ERR_INVALID_ARG;
    QH_TRY(hipMemsetAsync(dst, value, bytes, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_stream_create(qh_stream* s) {
    if (!s) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    hipStream_t st;
    QH_TRY(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = (qh_stream)st;
    return Q_OK;
}

q_error_code qh_stream_destroy(qh_stream s) {
    if (!s) return Q_OK;
    QH_TRY(hipStreamDestroy((hipStream_t)s));
    return Q_OK;
}

q_error_code qh_stream_synchronize(qh_stream s) {
    QH_TRY(hipStreamSynchronize((hipStream_t)s));
    return Q_OK;
}

q_error_code qh_device_synchronize(void) {
    QH_TRY(hipDeviceSynchronize());
    return Q_OK;
}

q_error_code qh_event_create(qh_event* e) {
    if (!e) return Q_ERR_INVALID_ARG;
    Device* d;
    QH_TRY_CODE(device(&d));
    hipEvent_t ev;
    QH_TRY(hipEventCreate(&ev));
    *e = (qh_event)ev;
    return Q_OK;
}

q_error_code qh_event_destroy(qh_event e) {
    if (!e) return Q_OK;
    QH_TRY(hipEventDestroy((hipEvent_t)e));
    return Q_OK;
}

q_error_code qh_event_record(qh_event e, qh_stream s) {
    if (!e) return Q_ERR_INVALID_ARG;
    QH_TRY(hipEventRecord((hipEvent_t)e, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_event_synchronize(qh_event e) {
    if (!e) return Q_ERR_INVALID_ARG;
    QH_TRY(hipEventSynchronize((hipEvent_t)e));
    return Q_OK;
}

q_error_code qh_event_elapsed_ms(qh_event start, qh_event stop, float* ms) {
    if (!start || !stop || !ms) return Q_ERR_INVALID_ARG;
    QH_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return Q_OK;
}

q_error_code qh_stream_begin_capture(qh_stream s) {
    if (!s) return Q_ERR_INVALID_ARG;  // the null stream cannot be captured
    QH_TRY(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal));
    return Q_OK;
}

q_error_code qh_stream_end_capture(qh_stream s, qh_graph* out) {
    if (!s || !out) return Q_ERR_INVALID_ARG;
    hipGraph_t g = nullptr;
    QH_TRY(hipStreamEndCapture((hipStream_t)s, &g));
    hipGraphExec_t ex = nullptr;
    const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail(e, "hipGraphInstantiate");
    *out = (qh_graph)ex;
    return Q_OK;
}

q_error_code qh_graph_launch(qh_graph g, qh_stream s) {
    if (!g) return Q_ERR_INVALID_ARG;
    QH_TRY(hipGraphLaunch((hipGraphExec_t)g, (hipStream_t)s));
    return Q_OK;
}

q_error_code qh_graph_destroy(qh_graph g) {
    if (!g) return Q_OK;
    QH_TRY(hipGraphExecDestroy((hipGraphExec_t)g));
    return Q_OK;
}

}  // extern "C"
