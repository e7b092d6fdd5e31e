/*
 * qorus_types.h -- ABI types of the Qorus-IA C API, re-declared for the
 * MI355X (gfx950) implementation.
 *
 * Every struct, enum and constant here is source- and binary-compatible with
 * the reference declaration it replaces (reference include/qorus_types.h).
 * Field order, widths, packing and alignment are part of the drop-in contract
 * and are pinned by the static assertions at the end of this file.
 *
 *   q_error_code    reference include/qorus_types.h:30-48
 *   q_mmap_strategy reference include/qorus_types.h:54-57
 *   q_dtype         reference include/qorus_types.h:134-138
 *   q_tokenizer     reference include/qorus_types.h:144-175 (type only)
 *   q_block_q4_0    reference include/qorus_types.h:181-186
 *   q_model_header  reference include/qorus_types.h:189-203
 *   q_tensor        reference include/qorus_types.h:205-213
 *   q_context       reference include/qorus_types.h:215-231
 *   q_llama_*       reference include/qorus_types.h:238-286
 *   q_generation_state reference include/qorus_types.h:293-306
 */
#ifndef QORUS_TYPES_H
#define QORUS_TYPES_H

#include <stdint.h>
#include <stddef.h>
#include <stdbool.h>

#define Q_ALIGN 64
#define Q_MAGIC 0x514F5231u /* 'QOR1' little-endian */
#define Q_HEADER_SIZE 64
#define Q_FIRST_TENSOR_OFFSET Q_HEADER_SIZE

/* Round a byte size up to the 64-byte tensor alignment of the .qorus file. */
#define Q_ALIGN_SIZE(size) (((size) + Q_ALIGN - 1) & ~((size_t)Q_ALIGN - 1))

/* Tolerances the reference test-suite compares against. */
#define Q_EPSILON_ABS_F32 1e-5f
#define Q_EPSILON_REL_F32 1e-4f
#define Q_EPSILON_ABS_APPROX 2.5e-1f
#define Q_EPSILON_REL_APPROX 5e-1f
#define Q_EPSILON_ABS_Q4_VAL 1e-2f
#define Q_EPSILON_REL_Q4_VAL 5e-2f

/* Return codes: 0 on success, negative on failure. */
typedef enum {
    Q_OK = 0,
    Q_ERR_NULL_PTR = -1,
    Q_ERR_FILE_OPEN = -2,
    Q_ERR_FILE_STAT = -3,
    Q_ERR_FILE_TOO_SMALL = -4,
    Q_ERR_MMAP_FAILED = -5,
    Q_ERR_INVALID_MAGIC = -6,
    Q_ERR_ALLOC_FAILED = -7,
    Q_ERR_ARENA_OOM = -8,
    Q_ERR_INVALID_CONFIG = -9,
    Q_ERR_INVALID_ARG = -10,
    Q_ERR_ALIASING = -11,
    Q_ERR_OVERFLOW = -12,
    Q_ERR_MISALIGNED = -13,
    Q_ERR_INVALID_DTYPE = -14,
    Q_ERR_INVALID_SIZE = -15
} q_error_code;

typedef enum {
    Q_MMAP_LAZY = 0,  /* map only; pages fault in on first touch */
    Q_MMAP_EAGER = 1  /* MAP_POPULATE */
} q_mmap_strategy;

typedef enum {
    Q_F32 = 0,
    Q_Q8_0 = 1,
    Q_Q4_0 = 2
} q_dtype;

/* BPE tokenizer state (q_tokenizer_load / encode / decode / free).
 * merge_hash_table is the library's own lookup table (opaque; NULL for a
 * tokenizer assembled by hand, whose rules then use merges[i].merged_id). */
typedef struct {
    uint32_t token_id1;
    uint32_t token_id2;
    uint32_t merged_id;
} q_bpe_merge;

struct bpe_hash_table;

typedef struct {
    char** vocab;
    uint32_t vocab_size;
    q_bpe_merge* merges;
    uint32_t num_merges;
    struct bpe_hash_table* merge_hash_table;
    uint32_t bos_token_id;
    uint32_t eos_token_id;
    uint32_t pad_token_id;
    bool initialized;
} q_tokenizer;

/*
 * One Q4_0 block: 32 weights in 20 bytes.
 * Element e of the block lives in byte qs[e >> 1]: the low nibble for even
 * e, the high nibble for odd e.  Its value is fmaf((float)nibble, scale,
 * -8.0f * scale), i.e. (nibble - 8) * scale.
 */
typedef struct {
    uint8_t qs[16];
    float scale;
} __attribute__((packed)) q_block_q4_0;

/* 64-byte file header of a .qorus model. */
typedef struct {
    uint32_t magic;
    uint32_t version;
    uint32_t vocab_size;
    uint32_t dim;
    uint32_t hidden_dim;
    uint32_t n_layers;
    uint32_t n_heads;
    uint32_t n_kv_heads;
    uint32_t max_seq_len;
    float rope_freq_base;
    float rms_norm_eps;
    uint32_t reserved[5];
} __attribute__((packed, aligned(64))) q_model_header;

/*
 * Tensor view.  For Q4_0 matrices ne[0] = rows (outputs), ne[1] = columns
 * (inputs, a multiple of 32) and nb[0] = ne[1] / 32 * 20 bytes.
 */
typedef struct {
    void* data;
    float* scales;
    uint32_t ne[4];
    size_t nb[4];
    q_dtype type;
    char name[32];
} __attribute__((aligned(Q_ALIGN))) q_tensor;

/*
 * Memory context: tier 1 = model weights (host mmap), tier 2 = KV cache,
 * tier 3 = bump arena.  In this build the KV cache is HBM-resident:
 * kv_buffer holds a device address.  The weights and the arena keep their
 * host meaning; their device mirrors live in a side table keyed by the
 * context address, so the struct layout is unchanged.
 */
typedef struct {
    void* weights_mmap;
    size_t weights_size;
    q_model_header* header;

    void* kv_buffer;
    size_t kv_size;

    void* scratch_buffer;
    size_t scratch_size;
    size_t scratch_head;
    size_t scratch_base_offset;
} q_context;

typedef struct {
    uint32_t vocab_size;
    uint32_t dim;
    uint32_t hidden_dim;
    uint32_t n_layers;
    uint32_t n_heads;
    uint32_t n_kv_heads;
    uint32_t max_seq_len;
    float rope_freq_base;
    float rms_norm_eps;
} q_llama_config;

typedef struct {
    uint32_t layer_idx;
    q_tensor* attn_norm;
    q_tensor* wq;
    q_tensor* wk;
    q_tensor* wv;
    q_tensor* wo;
    q_tensor* ffn_norm;
    q_tensor* w_gate;
    q_tensor* w_up;
    q_tensor* w_down;
} q_llama_layer;

typedef struct {
    q_llama_config config;
    q_tensor* token_embd;
    q_tensor* output_norm;
    q_tensor* output;
    q_llama_layer* layers;
    float* rope_freqs;
    bool rope_cache_enabled;
    float* rope_cos_cache;
    float* rope_sin_cache;
    q_context* ctx;
} q_llama_model;

typedef struct {
    q_context* ctx;
    q_llama_model* model;
    q_tokenizer* tokenizer;
    uint32_t* prompt_tokens;
    uint32_t num_prompt_tokens;
    uint32_t* generated_tokens;
    uint32_t num_generated_tokens;
    uint32_t max_tokens;
    float temperature;
    uint32_t top_k;
    float top_p;
    uint32_t current_pos;
} q_generation_state;

/* Layout pins (the reference ABI on x86-64 / LP64). */
#ifdef __cplusplus
#define Q_STATIC_ASSERT static_assert
#else
#define Q_STATIC_ASSERT _Static_assert
#endif
Q_STATIC_ASSERT(sizeof(q_block_q4_0) == 20, "q_block_q4_0 must be 20 bytes");
Q_STATIC_ASSERT(offsetof(q_block_q4_0, scale) == 16, "scale follows qs");
Q_STATIC_ASSERT(sizeof(q_model_header) == 64, "header is 64 bytes");
Q_STATIC_ASSERT(offsetof(q_tensor, data) == 0, "q_tensor.data");
Q_STATIC_ASSERT(offsetof(q_tensor, scales) == 8, "q_tensor.scales");
Q_STATIC_ASSERT(offsetof(q_tensor, ne) == 16, "q_tensor.ne");
Q_STATIC_ASSERT(offsetof(q_tensor, nb) == 32, "q_tensor.nb");
Q_STATIC_ASSERT(offsetof(q_tensor, type) == 64, "q_tensor.type");
Q_STATIC_ASSERT(offsetof(q_tensor, name) == 68, "q_tensor.name");
Q_STATIC_ASSERT(sizeof(q_tensor) == 128, "q_tensor is 128 bytes");
Q_STATIC_ASSERT(sizeof(q_context) == 72, "q_context is 72 bytes");

#endif /* QORUS_TYPES_H */
