// model.cpp -- Llama-3 decode on one MI355X behind the reference model API
// (llama_build_graph / llama_forward / llama_free_graph / q_sample_token).
//
// Host side keeps the reference's data structures: tensor views and layer
// structs in the q_context arena, pointing into the mapped .qorus file
// (reference src/models/model.c:294-673).  The device plan lives in the
// q_context side table: device addresses of every tensor (the HBM mirror
// made by q_init_memory, same offsets), one HBM scratch arena allocated once
// here (no allocation per token), RoPE tables for every position computed on
// the host with the reference's libm calls and uploaded, and a captured HIP
// graph of the whole decode step.  Token and position are read by the
// kernels from device memory, so the one graph serves every step and a
// generation loop can feed the greedy token back on the device.
//
// Model file: .qorus version 3 (shapes [out, in] as the GEMV consumes them,
// Q4_0 LM head); see qorus_amd/model_file.py.  The reference's own writer
// stores FP32 bytes in Q4_0 slots and [in, out] shapes, which its forward
// cannot run at Llama-3 shapes; those files are rejected with
// Q_ERR_INVALID_CONFIG.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "qh_decode.hpp"
#include "qh_kernels.hpp"
#include "qh_prefill.hpp"
#include "qh_runtime.hpp"
#include "qh_sample.hpp"

namespace qh {


struct LayerDev {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *attn_norm, *ffn_norm;
};

struct ModelPlan {
    const q_llama_model* model = nullptr;
    q_llama_config cfg{};
    uint32_t hd = 0, kvd = 0;
    float scale = 0.0f;
    const float* embd = nullptr;
    const float* out_norm = nullptr;
    const uint8_t* lm_head = nullptr;
    std::vector<LayerDev> layers;
    // HBM scratch arena (one allocation)
    uint8_t* arena = nullptr;
    size_t arena_bytes = 0;
    float *x = nullptr, *x1 = nullptr, *q = nullptr, *g = nullptr, *u = nullptr, *logits = nullptr;
    uint4 *xd_a = nullptr, *xd_b = nullptr, *xd_c = nullptr;
    float *scores = nullptr, *part_max = nullptr, *part_sum = nullptr, *o_part = nullptr;
    float *cos_tab = nullptr, *sin_tab = nullptr;
    uint32_t *tok = nullptr, *pos = nullptr, *hist = nullptr, *hist_n = nullptr;
    uint32_t hist_cap = 0;
    float* amax_ws = nullptr;                // multi-workgroup argmax partials
    float* amax_parts = nullptr;             // the LM-head GEMV's argmax partials
    bool fused = false;                      // 7-kernel layers (fp32-input GEMVs with fused prologues)
    float* kv = nullptr;
    size_t kv_layer_floats = 0;
    hipStream_t stream = nullptr;
    hipGraphExec_t step_graph = nullptr;     // decode step, host-fed token/pos
    hipGraphExec_t gen_graph = nullptr;      // decode step + greedy feedback + pos advance
    void* sample_ws = nullptr;               // device workspace of sampled generation
    uint32_t* pinned = nullptr;              // host staging for token/pos
    float* pinned_logits = nullptr;          // host staging for the logits llama_forward returns
    // Batched prefill (llama_forward with seq_len > 1), allocated at its
    // first use: row buffers for pf_rows tokens and the GEMM workspace.
    uint8_t* pf_arena = nullptr;
    uint32_t pf_rows = 0;
    float *pf_x = nullptr, *pf_x1 = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
    float *pf_o = nullptr, *pf_g = nullptr, *pf_u = nullptr;
    uint32_t* pf_tok = nullptr;
    void* pf_ws = nullptr;
    void* pf_khl = nullptr;  // the prefill attention's fp16 hi/lo key rows (one layer)
    uint32_t* pinned_tok = nullptr;          // host staging for a chunk's tokens
};

static std::mutex g_plan_mu;

void plan_destroy(CtxState* st) {
    std::lock_guard<std::mutex> lk(g_plan_mu);
    ModelPlan* p = static_cast<ModelPlan*>(st->plan);
    if (!p) return;
    if (p->stream) (void)hipStreamSynchronize(p->stream);
    if (p->step_graph) (void)hipGraphExecDestroy(p->step_graph);
    if (p->gen_graph) (void)hipGraphExecDestroy(p->gen_graph);
    if (p->arena) (void)hipFree(p->arena);
    if (p->sample_ws) (void)hipFree(p->sample_ws);
    if (p->pf_arena) (void)hipFree(p->pf_arena);
    if (p->pinned_tok) (void)hipHostFree(p->pinned_tok);
    if (p->pinned) (void)hipHostFree(p->pinned);
    if (p->pinned_logits) (void)hipHostFree(p->pinned_logits);
    if (p->stream) (void)hipStreamDestroy(p->stream);
    delete p;
    st->plan = nullptr;
    st->dev_arena = nullptr;
    st->dev_arena_size = 0;
}

// ---------------------------------------------------------------------------
// Host-side views (reference create_tensor_view, model.c:170-292)
// ---------------------------------------------------------------------------
static bool mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > SIZE_MAX / a) return false;
    *out = a * b;
    return true;
}

static size_t f32_bytes(uint32_t n0, uint32_t n1) {
    size_t s;
    if (!mul_ok(n0, n1, &s) || !mul_ok(s, 4, &s)) return 0;
    return s;
}

static size_t q4_bytes(uint32_t rows, uint32_t cols) {
    if (cols % 32 != 0) return 0;
    size_t s;
    if (!mul_ok(rows, cols / 32, &s) || !mul_ok(s, sizeof(q_block_q4_0), &s)) return 0;
    return s;
}

static q_tensor* make_view(q_context* ctx, size_t offset, uint32_t n0, uint32_t n1, q_dtype type, const char* name) {
    q_tensor* t = static_cast<q_tensor*>(q_arena_alloc(ctx, sizeof(q_tensor)));
    if (!t) return nullptr;
    std::memset(t, 0, sizeof(*t));
    t->data = static_cast<uint8_t*>(ctx->weights_mmap) + offset;
    t->scales = nullptr;
    t->ne[0] = n0;
    t->ne[1] = n1;
    t->ne[2] = 1;
    t->ne[3] = 1;
    t->type = type;
    if (type == Q_F32) {
        t->nb[3] = 4;
        t->nb[2] = 4;
        t->nb[1] = 4;
        t->nb[0] = (size_t)n1 * 4;
    } else {
        t->nb[0] = (size_t)(n1 / 32) * sizeof(q_block_q4_0);
        t->nb[1] = t->nb[2] = t->nb[3] = sizeof(q_block_q4_0);
    }
    std::strncpy(t->name, name, sizeof(t->name) - 1);
    return t;
}

// ---------------------------------------------------------------------------
// Decode step enqueue (all kernels on p->stream)
// ---------------------------------------------------------------------------
// One decode step in 7 kernels per layer: Q|K|V from fp32 x (RMSNorm and
// digits in the prologue, RoPE and KV-cache stores in the epilogue),
// attention (3 kernels: the reference's clamped polynomial exp needs the
// global max before any exponential; the combine emits o's digits), Wo +
// residual, W_gate|W_up from fp32 x1 (FFN RMSNorm in the prologue, SwiGLU
// in the epilogue, fp32 h out), W_down from fp32 h + residual.
static hipError_t enqueue_step_fused(ModelPlan* p, bool feedback) {
    const q_llama_config& c = p->cfg;
    hipStream_t s = p->stream;
    hipError_t e;
#define QH_E(x)                          \
    do {                                 \
        e = (x);                         \
        if (e != hipSuccess) return e;   \
    } while (0)
    const uint32_t nblk_d = c.dim / 32;
    QH_E(launch_embed(p->embd, p->tok, c.vocab_size, c.dim, p->x, s));
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const LayerDev& L = p->layers[l];
        float* kvl = p->kv + (size_t)l * p->kv_layer_floats;
        // Q|K|V of RMSNorm(x): the norm and the digits of x*attn_norm are
        // made in the GEMV's prologue; RoPE and the KV-cache stores in its
        // epilogue.
        GemvSeg qkv[3];
        qkv[0] = GemvSeg{L.wq, p->q, nullptr, c.dim};
        qkv[0].hd = p->hd;
        qkv[0].head_stride = p->hd;
        qkv[0].rope = true;
        qkv[1] = GemvSeg{L.wk, kvl, nullptr, p->kvd};
        qkv[1].hd = p->hd;
        qkv[1].head_stride = c.max_seq_len * 2 * p->hd;
        qkv[1].pos_stride = 2 * p->hd;
        qkv[1].rope = true;
        qkv[2] = GemvSeg{L.wv, kvl + p->hd, nullptr, p->kvd};
        qkv[2].hd = p->hd;
        qkv[2].head_stride = c.max_seq_len * 2 * p->hd;
        qkv[2].pos_stride = 2 * p->hd;
        GemvDecode dq;
        dq.pos = p->pos;
        dq.cos_tab = p->cos_tab;
        dq.sin_tab = p->sin_tab;
        dq.norm_w = L.attn_norm;
        dq.eps = c.rms_norm_eps;
        QH_E(launch_gemv_f32(qkv, 3, c.dim, p->x, nullptr, s, &dq));
        AttnArgs aa;
        aa.q = p->q;
        aa.kv_layer = kvl;
        aa.pos = p->pos;
        aa.n_heads = c.n_heads;
        aa.n_kv = c.n_kv_heads;
        aa.head_dim = p->hd;
        aa.max_seq = c.max_seq_len;
        aa.scale = p->scale;
        aa.scores = p->scores;
        aa.part_max = p->part_max;
        aa.part_sum = p->part_sum;
        aa.o_part = p->o_part;
        aa.o_out = nullptr;
        aa.xd_out = p->xd_b;
        QH_E(launch_attention(aa, s));
        // Wo + residual on the attention output's digits.
        GemvSeg wo{L.wo, p->x1, p->x, c.dim};
        QH_E(launch_gemv(&wo, 1, nblk_d, p->xd_b, s));
        // h = silu(W_gate.n) * (W_up.n), n = RMSNorm(x1) made in the prologue.
        QH_E(launch_gemv_swiglu(L.wg, L.wu, c.hidden_dim, c.dim, p->x1, L.ffn_norm, c.rms_norm_eps, p->g, s));
        // W_down + residual straight from the fp32 h.
        GemvSeg wd{L.wd, p->x, p->x1, c.dim};
        QH_E(launch_gemv_f32(&wd, 1, c.hidden_dim, p->g, nullptr, s));
    }
    // LM head of RMSNorm(x), the norm made in the GEMV's prologue.
    GemvDecode dn;
    dn.norm_w = p->out_norm;
    dn.eps = c.rms_norm_eps;
    GemvSeg lm{p->lm_head, p->logits, nullptr, c.vocab_size};
    // Greedy feedback: the LM-head GEMV also leaves the argmax's partials,
    // so the argmax is one small combine launch (where the shape allows).
    uint32_t n_part = 0;
    const hipError_t ea = feedback ? launch_gemv_f32_amax(lm, c.dim, p->x, &dn, p->amax_parts, kGemvAmaxMaxParts,
                                                          &n_part, s)
                                   : hipErrorNotSupported;
    if (ea == hipSuccess) {
        QH_E(launch_argmax_parts(p->logits, c.vocab_size, p->amax_parts, n_part, p->tok, p->pos, p->hist, p->hist_n,
                                 p->hist_cap, s));
    } else if (ea == hipErrorNotSupported) {
        QH_E(launch_gemv_f32(&lm, 1, c.dim, p->x, nullptr, s, &dn));
        if (feedback)
            QH_E(launch_argmax_ws(p->logits, c.vocab_size, p->tok, p->pos, p->hist, p->hist_n, p->hist_cap,
                                  p->amax_ws, s));
    } else {
        QH_E(ea);
    }
#undef QH_E
    return hipSuccess;
}

static hipError_t enqueue_step(ModelPlan* p, bool feedback) {
    if (p->fused) return enqueue_step_fused(p, feedback);
    const q_llama_config& c = p->cfg;
    hipStream_t s = p->stream;
    hipError_t e;
#define QH_E(x)                          \
    do {                                 \
        e = (x);                         \
        if (e != hipSuccess) return e;   \
    } while (0)
    QH_E(launch_embed(p->embd, p->tok, c.vocab_size, c.dim, p->x, s));
    GemvDecode dec;
    dec.pos = p->pos;
    dec.cos_tab = p->cos_tab;
    dec.sin_tab = p->sin_tab;
    const uint32_t nblk_d = c.dim / 32, nblk_h = c.hidden_dim / 32;
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const LayerDev& L = p->layers[l];
        float* kvl = p->kv + (size_t)l * p->kv_layer_floats;
        // attention block
        QH_E(launch_xprep(p->x, c.dim, L.attn_norm, c.rms_norm_eps, nullptr, p->xd_a, s));
        GemvSeg qkv[3];
        qkv[0] = GemvSeg{L.wq, p->q, nullptr, c.dim};
        qkv[0].hd = p->hd;
        qkv[0].head_stride = p->hd;
        qkv[0].rope = true;
        qkv[1] = GemvSeg{L.wk, kvl, nullptr, p->kvd};
        qkv[1].hd = p->hd;
        qkv[1].head_stride = c.max_seq_len * 2 * p->hd;
        qkv[1].pos_stride = 2 * p->hd;
        qkv[1].rope = true;
        qkv[2] = GemvSeg{L.wv, kvl + p->hd, nullptr, p->kvd};
        qkv[2].hd = p->hd;
        qkv[2].head_stride = c.max_seq_len * 2 * p->hd;
        qkv[2].pos_stride = 2 * p->hd;
        QH_E(launch_gemv(qkv, 3, nblk_d, p->xd_a, s, &dec));
        AttnArgs aa;
        aa.q = p->q;
        aa.kv_layer = kvl;
        aa.pos = p->pos;
        aa.n_heads = c.n_heads;
        aa.n_kv = c.n_kv_heads;
        aa.head_dim = p->hd;
        aa.max_seq = c.max_seq_len;
        aa.scale = p->scale;
        aa.scores = p->scores;
        aa.part_max = p->part_max;
        aa.part_sum = p->part_sum;
        aa.o_part = p->o_part;
        aa.o_out = nullptr;
        aa.xd_out = p->xd_b;
        QH_E(launch_attention(aa, s));
        GemvSeg wo{L.wo, p->x1, p->x, c.dim};
        QH_E(launch_gemv(&wo, 1, nblk_d, p->xd_b, s));
        // MLP block
        QH_E(launch_xprep(p->x1, c.dim, L.ffn_norm, c.rms_norm_eps, nullptr, p->xd_a, s));
        GemvSeg gu[2] = {GemvSeg{L.wg, p->g, nullptr, c.hidden_dim}, GemvSeg{L.wu, p->u, nullptr, c.hidden_dim}};
        QH_E(launch_gemv(gu, 2, nblk_d, p->xd_a, s));
        QH_E(launch_swiglu_prep(p->g, p->u, c.hidden_dim, nullptr, p->xd_c, s));
        GemvSeg wd{L.wd, p->x, p->x1, c.dim};
        QH_E(launch_gemv(&wd, 1, nblk_h, p->xd_c, s));
    }
    QH_E(launch_xprep(p->x, c.dim, p->out_norm, c.rms_norm_eps, nullptr, p->xd_a, s));
    GemvSeg lm{p->lm_head, p->logits, nullptr, c.vocab_size};
    QH_E(launch_gemv(&lm, 1, nblk_d, p->xd_a, s));
    if (feedback)
        QH_E(launch_argmax_ws(p->logits, c.vocab_size, p->tok, p->pos, p->hist, p->hist_n, p->hist_cap, p->amax_ws, s));
#undef QH_E
    return hipSuccess;
}

static q_error_code capture(ModelPlan* p, bool feedback, hipGraphExec_t* out) {
    QH_TRY(hipStreamBeginCapture(p->stream, hipStreamCaptureModeThreadLocal));
    const hipError_t e = enqueue_step(p, feedback);
    hipGraph_t g = nullptr;
    const hipError_t e2 = hipStreamEndCapture(p->stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return fail(e, "decode step capture");
    }
    if (e2 != hipSuccess) return fail(e2, "hipStreamEndCapture");
    const hipError_t e3 = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e3 != hipSuccess) return fail(e3, "hipGraphInstantiate");
    return Q_OK;
}

// ---------------------------------------------------------------------------
// Batched prefill: T tokens at positions pos0 .. pos0+T-1 through every layer
// as GEMMs on the matrix cores, the same result as T decode steps (see
// k_prefill.hip).  Per layer: Q|K|V = W . RMSNorm(X) (the norm made where the
// GEMM converts its rows), RoPE + KV-cache stores, causal attention over the
// cache, X1 = X + Wo . O, G|U = W . RMSNorm(X1), X = X1 + W_down .
// (silu(G) * U) (the SwiGLU product made where the GEMM converts its rows).
// The last chunk ends with the LM head of its last row.
// ---------------------------------------------------------------------------
constexpr uint32_t kPrefillRows = 2048;  // tokens per prefill chunk

static size_t prefill_ws_bytes(const ModelPlan* p, uint32_t T) {
    const q_llama_config& c = p->cfg;
    size_t b = gemm_workspace_bytes(c.dim, T, c.dim + 2 * p->kvd);
    b = std::max(b, gemm_workspace_bytes(c.dim, T, c.dim));
    b = std::max(b, gemm_workspace_bytes(c.dim, T, 2 * c.hidden_dim));
    b = std::max(b, gemm_workspace_bytes(c.hidden_dim, T, c.dim));
    return b;
}

static q_error_code prefill_alloc(ModelPlan* p) {
    if (p->pf_arena) return Q_OK;
    const q_llama_config& c = p->cfg;
    const uint32_t R = std::min(kPrefillRows, c.max_seq_len);
    size_t ws = 0;
    for (uint32_t T = 1; T <= R; ++T) ws = std::max(ws, prefill_ws_bytes(p, T));
    size_t bytes = 0;
    auto carve = [&](size_t b) {
        const size_t at = bytes;
        bytes += (b + 255) & ~(size_t)255;
        return at;
    };
    const size_t rd = (size_t)R * c.dim * 4, rk = (size_t)R * p->kvd * 4, rh = (size_t)R * c.hidden_dim * 4;
    const size_t o_x = carve(rd), o_x1 = carve(rd), o_q = carve(rd), o_k = carve(rk), o_v = carve(rk);
    const size_t o_o = carve(rd), o_g = carve(rh), o_u = carve(rh), o_t = carve((size_t)R * 4), o_ws = carve(ws);
    const size_t o_kh = carve(prefill_khl_bytes(c.n_kv_heads, c.max_seq_len));
    if (!p->pinned_tok)
        QH_TRY(hipHostMalloc(reinterpret_cast<void**>(&p->pinned_tok), (size_t)R * 4, hipHostMallocDefault));
    QH_TRY(hipMalloc(&p->pf_arena, bytes));
    uint8_t* A = p->pf_arena;
    p->pf_x = reinterpret_cast<float*>(A + o_x);
    p->pf_x1 = reinterpret_cast<float*>(A + o_x1);
    p->pf_q = reinterpret_cast<float*>(A + o_q);
    p->pf_k = reinterpret_cast<float*>(A + o_k);
    p->pf_v = reinterpret_cast<float*>(A + o_v);
    p->pf_o = reinterpret_cast<float*>(A + o_o);
    p->pf_g = reinterpret_cast<float*>(A + o_g);
    p->pf_u = reinterpret_cast<float*>(A + o_u);
    p->pf_tok = reinterpret_cast<uint32_t*>(A + o_t);
    p->pf_ws = A + o_ws;
    p->pf_khl = A + o_kh;
    p->pf_rows = R;
    return Q_OK;
}

static hipError_t enqueue_prefill(ModelPlan* p, uint32_t T, uint32_t pos0, bool last) {
    const q_llama_config& c = p->cfg;
    hipStream_t s = p->stream;
    hipError_t e;
#define QH_E(x)                          \
    do {                                 \
        e = (x);                         \
        if (e != hipSuccess) return e;   \
    } while (0)
    QH_E(launch_embed_rows(p->embd, p->pf_tok, T, c.dim, p->pf_x, s));
    // A split-K GEMM writing the residual stream (Wo, W_down) leaves its
    // reduction to the next GEMM's row conversion (the RMSNorm before
    // W_gate|W_up, and before the next layer's Q|K|V).
    GemmDeferred pend;
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const LayerDev& L = p->layers[l];
        float* kvl = p->kv + (size_t)l * p->kv_layer_floats;
        GemmSegs qkv;
        qkv.n = 3;
        qkv.w[0] = L.wq;
        qkv.w[1] = L.wk;
        qkv.w[2] = L.wv;
        qkv.y[0] = p->pf_q;
        qkv.y[1] = p->pf_k;
        qkv.y[2] = p->pf_v;
        qkv.M[0] = c.dim;
        qkv.M[1] = qkv.M[2] = p->kvd;
        GemmRows xn;
        xn.x = p->pf_x;
        xn.norm_w = L.attn_norm;
        xn.eps = c.rms_norm_eps;
        xn.T = T;
        xn.N = c.dim;
        xn.from = &pend;
        GemmDeferred qkv_part;  // the Q|K|V reduction is left to the RoPE pass
        QH_E(launch_gemm_ex(qkv, xn, p->pf_ws, s, &qkv_part));
        if (qkv_part.valid)
            QH_E(launch_rope_kv_rows(p->pf_q, nullptr, nullptr, p->cos_tab, p->sin_tab, pos0, T, c.n_heads,
                                     c.n_kv_heads, c.max_seq_len, kvl, s, qkv_part.part, qkv_part.split,
                                     qkv_part.meta));
        else
            QH_E(launch_rope_kv_rows(p->pf_q, p->pf_k, p->pf_v, p->cos_tab, p->sin_tab, pos0, T, c.n_heads,
                                     c.n_kv_heads, c.max_seq_len, kvl, s));
        PrefillAttnArgs aa;
        aa.q = p->pf_q;
        aa.kv = kvl;
        aa.o = p->pf_o;
        aa.T = T;
        aa.pos0 = pos0;
        aa.n_heads = c.n_heads;
        aa.n_kv = c.n_kv_heads;
        aa.max_seq = c.max_seq_len;
        aa.scale = p->scale;
        aa.khl = p->pf_khl;
        QH_E(launch_prefill_attention(aa, s));
        GemmSegs wo;
        wo.n = 1;
        wo.w[0] = L.wo;
        wo.y[0] = p->pf_x1;
        wo.res[0] = p->pf_x;
        wo.M[0] = c.dim;
        GemmRows on;
        on.x = p->pf_o;
        on.T = T;
        on.N = c.dim;
        QH_E(launch_gemm_ex(wo, on, p->pf_ws, s, &pend));
        GemmSegs gu;
        gu.n = 2;
        gu.w[0] = L.wg;
        gu.w[1] = L.wu;
        gu.y[0] = p->pf_g;
        gu.y[1] = p->pf_u;
        gu.M[0] = gu.M[1] = c.hidden_dim;
        GemmRows x1n;
        x1n.x = p->pf_x1;
        x1n.norm_w = L.ffn_norm;
        x1n.eps = c.rms_norm_eps;
        x1n.T = T;
        x1n.N = c.dim;
        x1n.from = &pend;
        QH_E(launch_gemm_ex(gu, x1n, p->pf_ws, s));
        GemmSegs wd;
        wd.n = 1;
        wd.w[0] = L.wd;
        wd.y[0] = p->pf_x;
        wd.res[0] = p->pf_x1;
        wd.M[0] = c.dim;
        GemmRows hn;
        hn.x = p->pf_g;
        hn.u = p->pf_u;
        hn.T = T;
        hn.N = c.hidden_dim;
        // The last layer's rows feed the LM head: reduced here.  So are they
        // when the next Q|K|V stages longer rows (dim > hidden_dim) than
        // W_down did: its staging would overwrite the partials it reads.
        const bool defer_down = l + 1 < c.n_layers && c.dim <= c.hidden_dim;
        QH_E(launch_gemm_ex(wd, hn, p->pf_ws, s, defer_down ? &pend : nullptr));
        if (!defer_down) pend.valid = false;
    }
    if (last) {
        // LM head of RMSNorm(last row), as in the decode step.
        const float* xr = p->pf_x + (size_t)(T - 1) * c.dim;
        GemvSeg lm{p->lm_head, p->logits, nullptr, c.vocab_size};
        if (p->fused) {
            GemvDecode dn;
            dn.norm_w = p->out_norm;
            dn.eps = c.rms_norm_eps;
            QH_E(launch_gemv_f32(&lm, 1, c.dim, xr, nullptr, s, &dn));
        } else {
            QH_E(launch_xprep(xr, c.dim, p->out_norm, c.rms_norm_eps, nullptr, p->xd_a, s));
            QH_E(launch_gemv(&lm, 1, c.dim / 32, p->xd_a, s));
        }
    }
#undef QH_E
    return hipSuccess;
}

static ModelPlan* plan_of(const q_llama_model* model, q_context* ctx) {
    CtxState* st = ctx_state(ctx, false);
    if (!st || !st->plan) return nullptr;
    ModelPlan* p = static_cast<ModelPlan*>(st->plan);
    return p->model == model ? p : nullptr;
}

static q_error_code check_kv(const ModelPlan* p, const q_context* ctx) {
    const size_t need = (size_t)p->cfg.n_layers * p->kv_layer_floats * sizeof(float);
    if (!ctx->kv_buffer || ctx->kv_size < need) return Q_ERR_INVALID_ARG;
    return Q_OK;
}

// The captured graphs embed the KV-cache address: re-capture if it moved.
static q_error_code bind_kv(ModelPlan* p, const q_context* ctx) {
    float* kv = static_cast<float*>(ctx->kv_buffer);
    if (p->kv != kv) {
        QH_TRY(hipStreamSynchronize(p->stream));
        if (p->step_graph) QH_TRY(hipGraphExecDestroy(p->step_graph));
        if (p->gen_graph) QH_TRY(hipGraphExecDestroy(p->gen_graph));
        p->step_graph = p->gen_graph = nullptr;
        p->kv = kv;
    }
    return Q_OK;
}

}  // namespace qh

using namespace qh;

extern "C" {

// Reference src/models/model.c:294-673 (validation order kept; version-3
// layout; the device plan added at the end).
q_error_code llama_build_graph(q_context* __restrict__ ctx, q_llama_model* __restrict__ model) {
    if (!ctx || !model) return Q_ERR_NULL_PTR;
    if (!ctx->weights_mmap || !ctx->header) return Q_ERR_NULL_PTR;
    const q_model_header* h = ctx->header;
    if (h->magic != Q_MAGIC) return Q_ERR_INVALID_MAGIC;
    if (h->n_layers == 0 || h->dim == 0 || h->vocab_size == 0 || h->n_heads == 0 || h->n_kv_heads == 0)
        return Q_ERR_INVALID_CONFIG;
    if (h->dim % 32 != 0 || h->hidden_dim % 32 != 0) return Q_ERR_INVALID_CONFIG;
    // This build: version-3 layout, GQA group dividing the heads, 128-wide
    // heads, d_model up to 16384 (the Q|K|V epilogue's persistent GEMV).
    if (h->version < 3 || h->hidden_dim == 0 || h->max_seq_len == 0) return Q_ERR_INVALID_CONFIG;
    if (h->dim / 32 > kGemvF32MaxBlk) return Q_ERR_INVALID_CONFIG;
    if (h->hidden_dim > 32768) return Q_ERR_INVALID_CONFIG;  // the prefill GEMM converts rows of N <= 32768
    const uint32_t group = h->n_kv_heads ? h->n_heads / h->n_kv_heads : 0;
    if (group != 1 && group != 2 && group != 4 && group != 8) return Q_ERR_INVALID_CONFIG;  // GQA groups built
    if (h->n_heads % h->n_kv_heads != 0 || h->dim % h->n_heads != 0 || h->dim / h->n_heads != 128)
        return Q_ERR_INVALID_CONFIG;
    CtxState* st = ctx_state(ctx, false);
    if (!st || !st->dev_weights) return Q_ERR_INVALID_ARG;  // not loaded by q_init_memory

    q_llama_config& cfg = model->config;
    cfg.vocab_size = h->vocab_size;
    cfg.dim = h->dim;
    cfg.hidden_dim = h->hidden_dim;
    cfg.n_layers = h->n_layers;
    cfg.n_heads = h->n_heads;
    cfg.n_kv_heads = h->n_kv_heads;
    cfg.max_seq_len = h->max_seq_len;
    cfg.rope_freq_base = h->rope_freq_base;
    cfg.rms_norm_eps = (h->version >= 2 && h->rms_norm_eps > 0.0f) ? h->rms_norm_eps : 1e-5f;
    model->ctx = ctx;
    const uint32_t hd = cfg.dim / cfg.n_heads;
    const uint32_t kvd = cfg.n_kv_heads * hd;

    // Tensor walk in file order, each tensor padded to 64 bytes.
    size_t off = Q_HEADER_SIZE;
    auto place = [&](size_t bytes, size_t* at) -> bool {
        if (bytes == 0) return false;
        const size_t al = Q_ALIGN_SIZE(bytes);
        if (al < bytes || off > ctx->weights_size || al > ctx->weights_size - off) return false;
        *at = off;
        off += al;
        return true;
    };
    size_t o;
    if (!place(f32_bytes(cfg.vocab_size, cfg.dim), &o)) return Q_ERR_INVALID_CONFIG;
    if (!(model->token_embd = make_view(ctx, o, cfg.vocab_size, cfg.dim, Q_F32, "token_embd.weight")))
        return Q_ERR_ARENA_OOM;
    if (!place(f32_bytes(cfg.dim, 1), &o)) return Q_ERR_INVALID_CONFIG;
    if (!(model->output_norm = make_view(ctx, o, cfg.dim, 1, Q_F32, "output_norm.weight"))) return Q_ERR_ARENA_OOM;
    if (!place(q4_bytes(cfg.vocab_size, cfg.dim), &o)) return Q_ERR_INVALID_CONFIG;
    if (!(model->output = make_view(ctx, o, cfg.vocab_size, cfg.dim, Q_Q4_0, "output.weight")))
        return Q_ERR_ARENA_OOM;
    model->layers = static_cast<q_llama_layer*>(q_arena_alloc(ctx, sizeof(q_llama_layer) * cfg.n_layers));
    if (!model->layers) return Q_ERR_ARENA_OOM;
    struct Spec {
        q_tensor** slot;
        uint32_t n0, n1;
        q_dtype type;
        const char* name;
    };
    for (uint32_t l = 0; l < cfg.n_layers; ++l) {
        q_llama_layer* L = &model->layers[l];
        std::memset(L, 0, sizeof(*L));
        L->layer_idx = l;
        const Spec specs[9] = {
            {&L->attn_norm, cfg.dim, 1, Q_F32, "attn_norm.weight"},
            {&L->wq, cfg.dim, cfg.dim, Q_Q4_0, "wq.weight"},
            {&L->wk, kvd, cfg.dim, Q_Q4_0, "wk.weight"},
            {&L->wv, kvd, cfg.dim, Q_Q4_0, "wv.weight"},
            {&L->wo, cfg.dim, cfg.dim, Q_Q4_0, "wo.weight"},
            {&L->ffn_norm, cfg.dim, 1, Q_F32, "ffn_norm.weight"},
            {&L->w_gate, cfg.hidden_dim, cfg.dim, Q_Q4_0, "w_gate.weight"},
            {&L->w_up, cfg.hidden_dim, cfg.dim, Q_Q4_0, "w_up.weight"},
            {&L->w_down, cfg.dim, cfg.hidden_dim, Q_Q4_0, "w_down.weight"},
        };
        for (const Spec& sp : specs) {
            const size_t bytes = sp.type == Q_F32 ? f32_bytes(sp.n0, sp.n1) : q4_bytes(sp.n0, sp.n1);
            if (!place(bytes, &o)) return Q_ERR_INVALID_CONFIG;
            if (!(*sp.slot = make_view(ctx, o, sp.n0, sp.n1, sp.type, sp.name))) return Q_ERR_ARENA_OOM;
        }
    }

    // RoPE (reference model.c:625-665): freq_i = powf(base, -2i/hd), tables
    // theta = freq_i * (float)pos through cosf/sinf, pairs duplicated.
    const uint32_t pairs = hd / 2;
    model->rope_freqs = static_cast<float*>(q_arena_alloc(ctx, pairs * sizeof(float)));
    if (!model->rope_freqs) return Q_ERR_ARENA_OOM;
    for (uint32_t i = 0; i < pairs; ++i) {
        const float fe = -2.0f * (float)i / (float)hd;
        model->rope_freqs[i] = powf(cfg.rope_freq_base, fe);
    }
    const size_t tab = (size_t)cfg.max_seq_len * hd;
    std::vector<float> heap_cos, heap_sin;
    float* ct = nullptr;
    float* sn = nullptr;
    model->rope_cache_enabled = false;
    model->rope_cos_cache = model->rope_sin_cache = nullptr;
    if (cfg.max_seq_len <= 8192) {
        model->rope_cos_cache = static_cast<float*>(q_arena_alloc(ctx, tab * sizeof(float)));
        model->rope_sin_cache = static_cast<float*>(q_arena_alloc(ctx, tab * sizeof(float)));
        if (model->rope_cos_cache && model->rope_sin_cache) model->rope_cache_enabled = true;
    }
    if (model->rope_cache_enabled) {
        ct = model->rope_cos_cache;
        sn = model->rope_sin_cache;
    } else {
        heap_cos.resize(tab);
        heap_sin.resize(tab);
        ct = heap_cos.data();
        sn = heap_sin.data();
    }
    for (uint32_t ps = 0; ps < cfg.max_seq_len; ++ps)
        for (uint32_t i = 0; i < pairs; ++i) {
            const float th = model->rope_freqs[i] * (float)ps;
            const float cv = cosf(th), sv = sinf(th);
            const size_t b = (size_t)ps * hd + 2 * i;
            ct[b] = cv;
            ct[b + 1] = cv;
            sn[b] = sv;
            sn[b + 1] = sv;
        }
    ctx->scratch_base_offset = ctx->scratch_head;

    // ---- device plan ----
    plan_destroy(st);
    ModelPlan* p = new ModelPlan();
    p->model = model;
    p->cfg = cfg;
    p->hd = hd;
    p->kvd = kvd;
    p->scale = 1.0f / sqrtf((float)hd);
    auto dev = [&](const q_tensor* t) -> const uint8_t* {
        return st->dev_weights + (static_cast<const uint8_t*>(t->data) - static_cast<const uint8_t*>(ctx->weights_mmap));
    };
    p->embd = reinterpret_cast<const float*>(dev(model->token_embd));
    p->out_norm = reinterpret_cast<const float*>(dev(model->output_norm));
    p->lm_head = dev(model->output);
    for (uint32_t l = 0; l < cfg.n_layers; ++l) {
        const q_llama_layer& L = model->layers[l];
        p->layers.push_back(LayerDev{dev(L.wq), dev(L.wk), dev(L.wv), dev(L.wo), dev(L.w_gate), dev(L.w_up),
                                     dev(L.w_down), reinterpret_cast<const float*>(dev(L.attn_norm)),
                                     reinterpret_cast<const float*>(dev(L.ffn_norm))});
    }
    p->kv_layer_floats = (size_t)cfg.n_kv_heads * cfg.max_seq_len * 2 * hd;
    p->hist_cap = cfg.max_seq_len;
    // HBM scratch arena layout (256-byte aligned pieces).
    size_t bytes = 0;
    auto carve = [&](size_t b) {
        const size_t at = bytes;
        bytes += (b + 255) & ~(size_t)255;
        return at;
    };
    const size_t o_x = carve(cfg.dim * 4), o_x1 = carve(cfg.dim * 4), o_q = carve(cfg.dim * 4);
    const size_t o_g = carve((size_t)cfg.hidden_dim * 4), o_u = carve((size_t)cfg.hidden_dim * 4);
    const size_t o_lg = carve((size_t)cfg.vocab_size * 4);
    const size_t o_xa = carve(xd_bytes(cfg.dim / 32)), o_xb = carve(xd_bytes(cfg.dim / 32));
    const size_t o_xc = carve(xd_bytes(cfg.hidden_dim / 32));
    const size_t nch = attention_n_chunks(cfg.max_seq_len);
    const size_t o_sc = carve((size_t)cfg.n_heads * cfg.max_seq_len * 4);
    const size_t o_pm = carve((size_t)cfg.n_heads * nch * 4), o_ps = carve((size_t)cfg.n_heads * nch * 4);
    const size_t o_op = carve(nch * cfg.n_heads * hd * 4);
    const size_t o_ct = carve(tab * 4), o_st = carve(tab * 4);
    const size_t o_tok = carve(4), o_pos = carve(4), o_hn = carve(4), o_hist = carve((size_t)p->hist_cap * 4);
    const size_t o_aw = carve(argmax_workspace_bytes(cfg.vocab_size));
    const size_t o_ap = carve((size_t)2 * kGemvAmaxMaxParts * 4);
    hipError_t e = hipMalloc(&p->arena, bytes);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&p->pinned), 64, hipHostMallocDefault);
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&p->pinned_logits), (size_t)cfg.vocab_size * 4, hipHostMallocDefault);
    if (e != hipSuccess) {
        fail(e, "decode plan allocation");
        st->plan = p;
        plan_destroy(st);
        return Q_ERR_ALLOC_FAILED;
    }
    p->arena_bytes = bytes;
    uint8_t* A = p->arena;
    p->x = reinterpret_cast<float*>(A + o_x);
    p->x1 = reinterpret_cast<float*>(A + o_x1);
    p->q = reinterpret_cast<float*>(A + o_q);
    p->g = reinterpret_cast<float*>(A + o_g);
    p->u = reinterpret_cast<float*>(A + o_u);
    p->logits = reinterpret_cast<float*>(A + o_lg);
    p->xd_a = reinterpret_cast<uint4*>(A + o_xa);
    p->xd_b = reinterpret_cast<uint4*>(A + o_xb);
    p->xd_c = reinterpret_cast<uint4*>(A + o_xc);
    p->scores = reinterpret_cast<float*>(A + o_sc);
    p->part_max = reinterpret_cast<float*>(A + o_pm);
    p->part_sum = reinterpret_cast<float*>(A + o_ps);
    p->o_part = reinterpret_cast<float*>(A + o_op);
    p->cos_tab = reinterpret_cast<float*>(A + o_ct);
    p->sin_tab = reinterpret_cast<float*>(A + o_st);
    p->tok = reinterpret_cast<uint32_t*>(A + o_tok);
    p->pos = reinterpret_cast<uint32_t*>(A + o_pos);
    p->hist_n = reinterpret_cast<uint32_t*>(A + o_hn);
    p->hist = reinterpret_cast<uint32_t*>(A + o_hist);
    p->amax_ws = reinterpret_cast<float*>(A + o_aw);
    p->amax_parts = reinterpret_cast<float*>(A + o_ap);
    p->fused = cfg.dim / 32 <= 128 && cfg.hidden_dim / 32 <= kGemvF32MaxBlk && (p->kvd % 32) == 0;
    st->plan = p;
    st->dev_arena = p->arena;
    st->dev_arena_size = bytes;
    e = hipMemset(p->arena, 0, bytes);
    if (e == hipSuccess) e = hipMemcpy(p->cos_tab, ct, tab * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->sin_tab, sn, tab * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        fail(e, "decode plan upload");
        plan_destroy(st);
        return Q_ERR_ALLOC_FAILED;
    }
    // Everything a later call needs is allocated here, so no llama_forward
    // (one token or a prompt) and no device generation loop allocates: the
    // prefill rows and GEMM workspace for chunks of up to 2048 tokens and the
    // sampler's workspace.
    q_error_code rc = prefill_alloc(p);
    if (rc == Q_OK) {
        const size_t wb = sample_workspace_bytes(cfg.vocab_size);
        e = wb ? hipMalloc(&p->sample_ws, wb) : hipErrorInvalidValue;
        if (e != hipSuccess) rc = fail(e, "sampler workspace");
    }
    if (rc != Q_OK) {
        plan_destroy(st);
        return Q_ERR_ALLOC_FAILED;
    }
    return Q_OK;
}

// Reference src/models/model.c:675-691 (plus the device plan).
void llama_free_graph(q_llama_model* __restrict__ model) {
    if (!model) return;
    if (model->ctx) {
        CtxState* st = ctx_state(model->ctx, false);
        if (st && st->plan && static_cast<ModelPlan*>(st->plan)->model == model) plan_destroy(st);
    }
    model->token_embd = nullptr;
    model->output_norm = nullptr;
    model->output = nullptr;
    model->layers = nullptr;
    model->ctx = nullptr;
    std::memset(&model->config, 0, sizeof(model->config));
}

// Reference src/models/model.c:1655-1850: tokens[0..seq_len) at positions
// pos.., logits of the last token copied to the host buffer `logits`, the KV
// cache filled at pos .. pos+seq_len-1.  One token runs the captured decode
// step; more run the batched prefill in chunks of up to 2048 tokens (the
// result of one decode step per token: causal attention over the cache).
q_error_code llama_forward(q_llama_model* __restrict__ model, q_context* __restrict__ ctx,
                           const uint32_t* __restrict__ tokens, uint32_t seq_len, uint32_t pos,
                           float* __restrict__ logits) {
    if (!model || !ctx || !tokens || !logits) return Q_ERR_INVALID_ARG;
    if (seq_len == 0) return Q_ERR_INVALID_SIZE;
    if (seq_len > model->config.max_seq_len) return Q_ERR_INVALID_SIZE;
    if (pos >= model->config.max_seq_len) return Q_ERR_INVALID_ARG;
    if (!ctx->scratch_buffer) return Q_ERR_INVALID_ARG;
    if (!ctx->kv_buffer) return Q_ERR_INVALID_ARG;
    if ((uint64_t)pos + seq_len > model->config.max_seq_len) return Q_ERR_INVALID_ARG;
    for (uint32_t t = 0; t < seq_len; ++t)
        if (tokens[t] >= model->config.vocab_size) return Q_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(g_plan_mu);
    ModelPlan* p = plan_of(model, ctx);
    if (!p) return Q_ERR_INVALID_ARG;
    QH_TRY_CODE(check_kv(p, ctx));
    QH_TRY_CODE(bind_kv(p, ctx));
    if (seq_len == 1) {
        if (!p->step_graph) QH_TRY_CODE(capture(p, false, &p->step_graph));
        QH_TRY(hipStreamSynchronize(p->stream));  // pinned staging is reused each step
        p->pinned[0] = tokens[0];
        p->pinned[1] = pos;
        QH_TRY(hipMemcpyAsync(p->tok, &p->pinned[0], 4, hipMemcpyHostToDevice, p->stream));
        QH_TRY(hipMemcpyAsync(p->pos, &p->pinned[1], 4, hipMemcpyHostToDevice, p->stream));
        QH_TRY(hipGraphLaunch(p->step_graph, p->stream));
    } else {
        QH_TRY_CODE(prefill_alloc(p));
        for (uint32_t c0 = 0; c0 < seq_len; c0 += p->pf_rows) {
            const uint32_t T = std::min(p->pf_rows, seq_len - c0);
            QH_TRY(hipStreamSynchronize(p->stream));  // the token staging is reused per chunk
            std::memcpy(p->pinned_tok, tokens + c0, (size_t)T * 4);
            QH_TRY(hipMemcpyAsync(p->pf_tok, p->pinned_tok, (size_t)T * 4, hipMemcpyHostToDevice, p->stream));
            const hipError_t e = enqueue_prefill(p, T, pos + c0, c0 + T == seq_len);
            if (e != hipSuccess) return fail(e, "llama_forward: prefill launch");
        }
    }
    // through pinned memory (one DMA, then a host copy): a pageable copy of
    // the 513 KB Llama-3 logits is several times slower
    QH_TRY(hipMemcpyAsync(p->pinned_logits, p->logits, (size_t)model->config.vocab_size * 4, hipMemcpyDeviceToHost,
                          p->stream));
    QH_TRY(hipStreamSynchronize(p->stream));
    std::memcpy(logits, p->pinned_logits, (size_t)model->config.vocab_size * 4);
    return Q_OK;
}

// Reference src/main.c:994-1131, validation in its order: NULL state, ctx,
// model, tokenizer, prompt_tokens or generated_tokens -> INVALID_ARG; no
// prompt tokens or max_tokens 0 -> INVALID_SIZE; temperature negative, NaN or
// infinite -> INVALID_ARG; tokenizer not initialized, no arena or no KV
// cache -> INVALID_ARG; a prompt longer than max_seq_len -> INVALID_SIZE.
// Then: the prompt at position 0, and per step a draw from the last logits
// (q_sample_token with the context's arena; the logits in 64-byte-aligned
// host memory, as the reference allocates them), a stop at EOS or a full
// context, the token forwarded at the next position; the arena is reset
// before each forward.
q_error_code q_generate(q_generation_state* __restrict__ st) {
    if (!st || !st->ctx || !st->model || !st->tokenizer || !st->prompt_tokens || !st->generated_tokens)
        return Q_ERR_INVALID_ARG;
    if (st->num_prompt_tokens == 0 || st->max_tokens == 0) return Q_ERR_INVALID_SIZE;
    if (!(st->temperature >= 0.0f) || !std::isfinite(st->temperature)) return Q_ERR_INVALID_ARG;
    if (!st->tokenizer->initialized) return Q_ERR_INVALID_ARG;
    if (!st->ctx->scratch_buffer || !st->ctx->kv_buffer) return Q_ERR_INVALID_ARG;
    const uint32_t V = st->model->config.vocab_size, max_seq = st->model->config.max_seq_len;
    if (st->num_prompt_tokens > max_seq) return Q_ERR_INVALID_SIZE;
    st->num_generated_tokens = 0;
    st->current_pos = 0;
    q_arena_reset(st->ctx);
    float* logits = static_cast<float*>(std::aligned_alloc(Q_ALIGN, Q_ALIGN_SIZE((size_t)V * sizeof(float))));
    if (!logits) return Q_ERR_ALLOC_FAILED;
    q_error_code rc = llama_forward(st->model, st->ctx, st->prompt_tokens, st->num_prompt_tokens, 0, logits);
    if (rc == Q_OK) st->current_pos = st->num_prompt_tokens;
    while (rc == Q_OK && st->num_generated_tokens < st->max_tokens && st->current_pos < max_seq) {
        uint32_t tok = 0;
        rc = q_sample_token(logits, V, st->temperature, st->top_k, st->top_p, &tok, st->ctx);
        if (rc != Q_OK) break;
        if (tok >= V) {
            rc = Q_ERR_INVALID_ARG;
            break;
        }
        st->generated_tokens[st->num_generated_tokens++] = tok;
        if (tok == st->tokenizer->eos_token_id) break;
        q_arena_reset(st->ctx);
        rc = llama_forward(st->model, st->ctx, &tok, 1, st->current_pos, logits);
        if (rc == Q_OK) ++st->current_pos;
    }
    std::free(logits);
    return rc;
}

// Greedy generation on the device: n_steps decode steps from (token, pos),
// each step's argmax fed back as the next token and the position advanced
// on the device (no host round trip between steps).  tokens_out (host,
// n_steps entries) receives the generated tokens; *ms_per_step the mean
// step time measured with HIP events over the n_steps graph replays.
q_error_code qh_llama_generate(q_llama_model* model, q_context* ctx, uint32_t token, uint32_t pos,
                               uint32_t n_steps, uint32_t* tokens_out, float* ms_per_step) {
    if (!model || !ctx || !tokens_out) return Q_ERR_INVALID_ARG;
    if (n_steps == 0) return Q_ERR_INVALID_SIZE;
    if (token >= model->config.vocab_size) return Q_ERR_INVALID_ARG;
    if ((uint64_t)pos + n_steps > model->config.max_seq_len) return Q_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(g_plan_mu);
    ModelPlan* p = plan_of(model, ctx);
    if (!p) return Q_ERR_INVALID_ARG;
    QH_TRY_CODE(check_kv(p, ctx));
    QH_TRY_CODE(bind_kv(p, ctx));
    if (!p->gen_graph) QH_TRY_CODE(capture(p, true, &p->gen_graph));
    QH_TRY(hipStreamSynchronize(p->stream));
    p->pinned[0] = token;
    p->pinned[1] = pos;
    p->pinned[2] = 0;
    QH_TRY(hipMemcpyAsync(p->tok, &p->pinned[0], 4, hipMemcpyHostToDevice, p->stream));
    QH_TRY(hipMemcpyAsync(p->pos, &p->pinned[1], 4, hipMemcpyHostToDevice, p->stream));
    QH_TRY(hipMemcpyAsync(p->hist_n, &p->pinned[2], 4, hipMemcpyHostToDevice, p->stream));
    hipEvent_t e0, e1;
    QH_TRY(hipEventCreate(&e0));
    QH_TRY(hipEventCreate(&e1));
    QH_TRY(hipEventRecord(e0, p->stream));
    for (uint32_t i = 0; i < n_steps; ++i) QH_TRY(hipGraphLaunch(p->gen_graph, p->stream));
    QH_TRY(hipEventRecord(e1, p->stream));
    QH_TRY(hipEventSynchronize(e1));
    float ms = 0.0f;
    QH_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (ms_per_step) *ms_per_step = ms / (float)n_steps;
    QH_TRY(hipMemcpy(tokens_out, p->hist, (size_t)n_steps * 4, hipMemcpyDeviceToHost));
    return Q_OK;
}

// Sampled generation on the device (the q_generate loop of reference
// src/main.c:994-1131 with temperature/top-k/top-p, tokenizer aside): each
// step is the captured decode step, then q_sample_token's device pipeline
// on the logits in HBM writing the next token straight into the step's
// token slot, then the history append and position advance.  The uniform
// draws come from the calling thread's stream (one per step, in order), so
// the tokens equal those of a host loop of llama_forward + q_sample_token
// on the same thread (with 32-byte-aligned host logits, as the reference's
// arena gives).  temperature < 1e-6 is the greedy qh_llama_generate.
q_error_code qh_llama_generate_sampled(q_llama_model* model, q_context* ctx, uint32_t token, uint32_t pos,
                                       uint32_t n_steps, float temperature, uint32_t top_k, float top_p,
                                       uint32_t* tokens_out, float* ms_per_step) {
    if (!(temperature >= 0.0f) || !std::isfinite(temperature)) return Q_ERR_INVALID_ARG;
    if (temperature < 1e-6f) return qh_llama_generate(model, ctx, token, pos, n_steps, tokens_out, ms_per_step);
    if (!model || !ctx || !tokens_out) return Q_ERR_INVALID_ARG;
    if (n_steps == 0) return Q_ERR_INVALID_SIZE;
    if (token >= model->config.vocab_size) return Q_ERR_INVALID_ARG;
    if ((uint64_t)pos + n_steps > model->config.max_seq_len) return Q_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(g_plan_mu);
    ModelPlan* p = plan_of(model, ctx);
    if (!p) return Q_ERR_INVALID_ARG;
    QH_TRY_CODE(check_kv(p, ctx));
    QH_TRY_CODE(bind_kv(p, ctx));
    if (!p->step_graph) QH_TRY_CODE(capture(p, false, &p->step_graph));
    const uint32_t V = p->cfg.vocab_size;
    if (!p->sample_ws) {
        const size_t wb = sample_workspace_bytes(V);
        if (wb == 0) return fail(hipErrorInvalidValue, "qh_llama_generate_sampled: workspace size");
        QH_TRY(hipMalloc(&p->sample_ws, wb));
    }
    SampleParams sp;
    sp.vocab = V;
    sp.temperature = temperature;
    sp.inv_temperature = 1.0f / temperature;
    sp.n_mul = V >= 8 ? (V & ~7u) : 0u;  // device logits are 256-byte aligned
    sp.top_k = top_k;
    sp.top_p = top_p;
    QH_TRY(hipStreamSynchronize(p->stream));
    p->pinned[0] = token;
    p->pinned[1] = pos;
    p->pinned[2] = 0;
    QH_TRY(hipMemcpyAsync(p->tok, &p->pinned[0], 4, hipMemcpyHostToDevice, p->stream));
    QH_TRY(hipMemcpyAsync(p->pos, &p->pinned[1], 4, hipMemcpyHostToDevice, p->stream));
    QH_TRY(hipMemcpyAsync(p->hist_n, &p->pinned[2], 4, hipMemcpyHostToDevice, p->stream));
    hipEvent_t e0, e1;
    QH_TRY(hipEventCreate(&e0));
    QH_TRY(hipEventCreate(&e1));
    QH_TRY(hipEventRecord(e0, p->stream));
    for (uint32_t i = 0; i < n_steps; ++i) {
        QH_TRY(hipGraphLaunch(p->step_graph, p->stream));
        sp.r = sample_draw();
        QH_TRY(launch_sample(p->logits, sp, p->sample_ws, p->tok, p->stream));
        QH_TRY(launch_token_feedback(p->tok, p->pos, p->hist, p->hist_n, p->hist_cap, p->stream));
    }
    QH_TRY(hipEventRecord(e1, p->stream));
    QH_TRY(hipEventSynchronize(e1));
    float ms = 0.0f;
    QH_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (ms_per_step) *ms_per_step = ms / (float)n_steps;
    QH_TRY(hipMemcpy(tokens_out, p->hist, (size_t)n_steps * 4, hipMemcpyDeviceToHost));
    return Q_OK;
}

}  // extern "C"
