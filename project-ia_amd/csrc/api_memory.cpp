// api_memory.cpp -- the three memory tiers of q_context on MI355X.
//
//  Tier 1 (weights): the .qorus file is mapped on the host exactly as the
//      reference does (views keep host addresses) and uploaded once into one
//      HBM allocation; device code addresses tensors at the same offsets.
//  Tier 2 (KV cache): one zero-filled HBM allocation; kv_buffer is a device
//      address.
//  Tier 3 (arena): the host bump arena of the reference (model views and
//      structs live there); the decode step's device scratch is a separate
//      HBM arena sized and allocated once by llama_build_graph.
// Nothing here runs in the per-token hot path.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "qh_runtime.hpp"

namespace qh {
void plan_destroy(CtxState* st);  // model.cpp
}

using namespace qh;

static size_t align64_checked(size_t size) {
    if (size > SIZE_MAX - (Q_ALIGN - 1)) return 0;
    return (size + Q_ALIGN - 1) & ~(size_t)(Q_ALIGN - 1);
}

extern "C" {

// Reference src/core/memory.c:60-128 (+ the HBM upload).
q_error_code q_init_memory_ex(q_context* __restrict__ ctx, const char* model_path, q_mmap_strategy strategy) {
    if (!ctx || !model_path) return Q_ERR_INVALID_ARG;
    const int fd = open(model_path, O_RDONLY);
    if (fd < 0) return Q_ERR_FILE_OPEN;
    struct stat sb;
    if (fstat(fd, &sb) < 0) {
        close(fd);
        return Q_ERR_FILE_STAT;
    }
    const size_t size = (size_t)sb.st_size;
    if (size < Q_HEADER_SIZE) {
        close(fd);
        return Q_ERR_FILE_TOO_SMALL;
    }
    int flags = MAP_PRIVATE;
    if (strategy == Q_MMAP_EAGER) flags |= MAP_POPULATE;
    void* map = mmap(nullptr, size, PROT_READ, flags, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return Q_ERR_MMAP_FAILED;
    madvise(map, size, MADV_SEQUENTIAL | MADV_WILLNEED);
    const q_model_header* h = static_cast<const q_model_header*>(map);
    if (h->magic != Q_MAGIC) {
        munmap(map, size);
        return Q_ERR_INVALID_MAGIC;
    }
    // HBM mirror of the whole file.
    Device* d = nullptr;
    q_error_code rc = device(&d);
    void* dev = nullptr;
    if (rc == Q_OK) {
        hipError_t e = hipMalloc(&dev, size);
        if (e == hipSuccess) e = hipMemcpy(dev, map, size, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            rc = fail(e, "upload of the model to HBM");
            if (dev) (void)hipFree(dev);
            rc = Q_ERR_ALLOC_FAILED;
        }
    }
    if (rc != Q_OK) {
        munmap(map, size);
        return rc;
    }
    ctx->weights_mmap = map;
    ctx->weights_size = size;
    ctx->header = static_cast<q_model_header*>(map);
    CtxState* st = ctx_state(ctx, true);
    st->dev_weights = static_cast<uint8_t*>(dev);
    st->weights_size = size;
    return Q_OK;
}

// Reference src/core/memory.c:131-133.
q_error_code q_init_memory(q_context* __restrict__ ctx, const char* model_path) {
    return q_init_memory_ex(ctx, model_path, Q_MMAP_LAZY);
}

// Reference src/core/memory.c:136-164, in HBM.
q_error_code q_alloc_kv_cache(q_context* __restrict__ ctx, size_t kv_size) {
    if (!ctx) return Q_ERR_INVALID_ARG;
    if (ctx->kv_buffer) return Q_ERR_INVALID_ARG;
    const size_t sz = align64_checked(kv_size);
    if (sz == 0) return Q_ERR_OVERFLOW;
    Device* d;
    if (device(&d) != Q_OK) return Q_ERR_ALLOC_FAILED;
    void* p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) return Q_ERR_ALLOC_FAILED;
    if (hipMemset(p, 0, sz) != hipSuccess) {
        (void)hipFree(p);
        return Q_ERR_ALLOC_FAILED;
    }
    ctx->kv_buffer = p;
    ctx->kv_size = sz;
    return Q_OK;
}

// Reference src/core/memory.c:168-195 (host arena).
q_error_code q_alloc_arena(q_context* __restrict__ ctx, size_t arena_size) {
    if (!ctx) return Q_ERR_INVALID_ARG;
    if (ctx->scratch_buffer) return Q_ERR_INVALID_ARG;
    const size_t sz = align64_checked(arena_size);
    if (sz == 0) return Q_ERR_OVERFLOW;
    void* p = aligned_alloc(Q_ALIGN, sz);
    if (!p) return Q_ERR_ALLOC_FAILED;
    ctx->scratch_buffer = p;
    ctx->scratch_size = sz;
    ctx->scratch_head = 0;
    ctx->scratch_base_offset = 0;
    return Q_OK;
}

// Reference src/core/memory.c:199-259.
void* q_arena_alloc(q_context* __restrict__ ctx, size_t size) {
    if (!ctx || !ctx->scratch_buffer) return nullptr;
    const size_t sz = align64_checked(size);
    if (sz == 0) return nullptr;
    if (ctx->scratch_head > SIZE_MAX - sz) return nullptr;
    const size_t nh = ctx->scratch_head + sz;
    if (nh > ctx->scratch_size) return nullptr;
    void* p = static_cast<uint8_t*>(ctx->scratch_buffer) + ctx->scratch_head;
    ctx->scratch_head = nh;
    return p;
}

// Reference src/core/memory.c:265-315 (release semantics).
void q_arena_reset(q_context* __restrict__ ctx) {
    if (!ctx) return;
    ctx->scratch_head = ctx->scratch_base_offset;
}

// Reference src/core/memory.c:317-355: arena, then KV, then weights (LIFO),
// plus the HBM mirrors held in the side table.
void q_free_memory(q_context* __restrict__ ctx) {
    if (!ctx) return;
    CtxState* st = ctx_state(ctx, false);
    if (st) {
        (void)hipDeviceSynchronize();
        plan_destroy(st);
        if (st->dev_arena) (void)hipFree(st->dev_arena);
        if (st->dev_weights) (void)hipFree(st->dev_weights);
        ctx_state_erase(ctx);
    }
    if (ctx->scratch_buffer) {
        free(ctx->scratch_buffer);
        ctx->scratch_buffer = nullptr;
        ctx->scratch_size = 0;
        ctx->scratch_head = 0;
        ctx->scratch_base_offset = 0;
    }
    if (ctx->kv_buffer) {
        (void)hipFree(ctx->kv_buffer);
        ctx->kv_buffer = nullptr;
        ctx->kv_size = 0;
    }
    if (ctx->weights_mmap) {
        munmap(ctx->weights_mmap, ctx->weights_size);
        ctx->weights_mmap = nullptr;
        ctx->weights_size = 0;
        ctx->header = nullptr;
    }
}

// Reference src/core/utils.c:11-31.  Callers pass any int (the reference's
// own tests pass codes outside the enum); the code is read as an int, since
// C++ gives an enum without a fixed type only its enumerators' range.
const char* q_strerror(q_error_code err) {
    static_assert(sizeof(q_error_code) == sizeof(int), "q_error_code is passed as an int");
    int code;
    std::memcpy(&code, &err, sizeof code);
    switch (code) {
        case Q_OK: return "Success";
        case Q_ERR_NULL_PTR: return "Null pointer argument";
        case Q_ERR_FILE_OPEN: return "Failed to open file";
        case Q_ERR_FILE_STAT: return "Failed to stat file";
        case Q_ERR_FILE_TOO_SMALL: return "File too small (corrupt header?)";
        case Q_ERR_MMAP_FAILED: return "mmap() failed";
        case Q_ERR_INVALID_MAGIC: return "Invalid file magic (not a Qorus file)";
        case Q_ERR_ALLOC_FAILED: return "Memory allocation failed";
        case Q_ERR_ARENA_OOM: return "Arena Out of Memory";
        case Q_ERR_INVALID_CONFIG: return "Invalid model configuration";
        case Q_ERR_INVALID_ARG: return "Invalid argument";
        case Q_ERR_ALIASING: return "Input/output aliasing detected";
        case Q_ERR_OVERFLOW: return "Integer overflow detected";
        case Q_ERR_MISALIGNED: return "Pointer not properly aligned";
        case Q_ERR_INVALID_DTYPE: return "Invalid data type";
        case Q_ERR_INVALID_SIZE: return "Invalid size";
    }
    return "Unknown error";
}

}  // extern "C"
