/*
 * generate -- end-to-end text generation through libqorus_hip.so: load a
 * .qorus v3 model (HBM-resident weights) and a 'QTKR' tokenizer, encode the
 * prompt, run q_generate (batched prefill, then one decode step per token,
 * sampling on the GPU), decode and print, with the time of each phase.
 *
 *   generate <model.qorus> <tokenizer.bin> "<prompt>" [max_tokens] [temperature] [top_k] [top_p]
 *
 * Defaults: 32 tokens, temperature 0 (greedy), top-k 0, top-p 0.
 */
#define _POSIX_C_SOURCE 199309L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "qorus.h"

static double now_ms(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e3 + (double)t.tv_nsec * 1e-6;
}

static int fail(const char* what, q_error_code e) {
    fprintf(stderr, "error: %s: %s\n", what, q_strerror(e));
    return 1;
}

int main(int argc, char** argv) {
    if (argc < 4) {
        fprintf(stderr, "usage: %s <model.qorus> <tokenizer.bin> \"<prompt>\" [max_tokens] [temperature] [top_k] [top_p]\n",
                argv[0]);
        return 2;
    }
    const uint32_t max_tokens = argc > 4 ? (uint32_t)strtoul(argv[4], NULL, 10) : 32u;
    const float temperature = argc > 5 ? strtof(argv[5], NULL) : 0.0f;
    const uint32_t top_k = argc > 6 ? (uint32_t)strtoul(argv[6], NULL, 10) : 0u;
    const float top_p = argc > 7 ? strtof(argv[7], NULL) : 0.0f;

    double t0 = now_ms();
    q_context ctx;
    memset(&ctx, 0, sizeof(ctx));
    q_error_code e = q_init_memory(&ctx, argv[1]);
    if (e != Q_OK) return fail("q_init_memory", e);
    /* KV cache and arena before llama_build_graph: the graph's tensor views
     * live in the arena. */
    const q_model_header* hd = ctx.header;
    const size_t kv = Q_ALIGN_SIZE((size_t)hd->n_layers * hd->n_kv_heads * hd->max_seq_len *
                                   (hd->dim / hd->n_heads) * 2 * sizeof(float));
    if ((e = q_alloc_kv_cache(&ctx, kv)) != Q_OK) return fail("q_alloc_kv_cache", e);
    if ((e = q_alloc_arena(&ctx, (size_t)64 << 20)) != Q_OK) return fail("q_alloc_arena", e);
    q_llama_model model;
    memset(&model, 0, sizeof(model));
    if ((e = llama_build_graph(&ctx, &model)) != Q_OK) return fail("llama_build_graph", e);
    const q_llama_config* c = &model.config;
    q_tokenizer tok;
    memset(&tok, 0, sizeof(tok));
    if ((e = q_tokenizer_load(&tok, argv[2])) != Q_OK) return fail("q_tokenizer_load", e);
    const double t_load = now_ms() - t0;

    const uint32_t cap = (uint32_t)strlen(argv[3]) + 2;
    uint32_t* prompt = malloc(sizeof(uint32_t) * cap);
    uint32_t* out = malloc(sizeof(uint32_t) * (max_tokens ? max_tokens : 1));
    uint32_t n_prompt = 0;
    if (!prompt || !out) return fail("malloc", Q_ERR_ALLOC_FAILED);
    if ((e = q_tokenizer_encode(&tok, argv[3], prompt, &n_prompt, cap, true, false)) != Q_OK)
        return fail("q_tokenizer_encode", e);

    q_generation_state st;
    memset(&st, 0, sizeof(st));
    st.ctx = &ctx;
    st.model = &model;
    st.tokenizer = &tok;
    st.prompt_tokens = prompt;
    st.num_prompt_tokens = n_prompt;
    st.generated_tokens = out;
    st.max_tokens = max_tokens;
    st.temperature = temperature;
    st.top_k = top_k;
    st.top_p = top_p;
    t0 = now_ms();
    if ((e = q_generate(&st)) != Q_OK) return fail("q_generate", e);
    const double t_gen = now_ms() - t0;

    size_t text_cap = 16;
    for (uint32_t i = 0; i < st.num_generated_tokens; ++i)
        if (out[i] < tok.vocab_size && tok.vocab[out[i]]) text_cap += strlen(tok.vocab[out[i]]);
    char* text = malloc(text_cap);
    if (!text) return fail("malloc", Q_ERR_ALLOC_FAILED);
    if ((e = q_tokenizer_decode(&tok, out, st.num_generated_tokens, text, text_cap)) != Q_OK)
        return fail("q_tokenizer_decode", e);

    printf("model: d_model %u, %u layers, %u heads (%u kv), vocab %u, context %u\n", c->dim, c->n_layers, c->n_heads,
           c->n_kv_heads, c->vocab_size, c->max_seq_len);
    printf("prompt tokens (%u):", n_prompt);
    for (uint32_t i = 0; i < n_prompt; ++i) printf(" %u", prompt[i]);
    printf("\ngenerated tokens (%u):", st.num_generated_tokens);
    for (uint32_t i = 0; i < st.num_generated_tokens; ++i) printf(" %u", out[i]);
    printf("\ngenerated text: \"%s\"\n", text);
    printf("load %.1f ms; generate %.2f ms for %u prompt + %u new tokens\n", t_load, t_gen, n_prompt,
           st.num_generated_tokens);

    free(text);
    free(out);
    free(prompt);
    q_tokenizer_free(&tok);
    llama_free_graph(&model);
    q_free_memory(&ctx);
    return 0;
}
