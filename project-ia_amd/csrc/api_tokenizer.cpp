// api_tokenizer.cpp -- the byte-level BPE tokenizer of the reference API
// (q_tokenizer_load / encode / decode / free, reference include/qorus.h:230-
// 273, src/tokenizer/bpe.c), host code.  Text enters and leaves the model as
// token ids; nothing here touches the GPU.
//
// File format (reference bpe.c:24-26, 263-...): a 32-byte little-endian
// header {magic 'QTKR' 0x51544B52, version 1, vocab_size, num_merges, bos,
// eos, pad, reserved}, then vocab_size entries {u8 length >= 1, bytes}, then
// num_merges rules {u32 token_id1, u32 token_id2, u32 merged_id}.
//
// Encoding (reference bpe.c:568-808): each byte of the text is a token (its
// value when below vocab_size, else the pad id); then, while anything
// changes, every merge rule in file order is applied to every adjacent live
// pair (a, b) == (id1, id2) from left to right (the pair becomes one token at
// a's place; the scan resumes after b, so a token made by a rule is paired by
// that rule again only on the next pass); BOS first / EOS last on request.
//
// The merged id used for rule i: a tokenizer built by q_tokenizer_load looks
// every rule up by the key (id1 << 16) | id2 in a table whose entries for
// equal keys answer with the last rule of that key in file order (the
// reference's chained hash table, insertion at the chain head).  Different
// pairs share a key when an id reaches 65536, so in a large vocabulary a rule
// can produce another rule's merged id; this build reproduces that.  A
// tokenizer assembled by hand (no table) uses merges[i].merged_id.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <unordered_map>
#include <vector>

#include "qorus.h"

// The table behind q_tokenizer.merge_hash_table: the merged id each rule
// produces (see above).
struct bpe_hash_table {
    std::vector<uint32_t> merged;
};

namespace {

constexpr uint32_t kTokMagic = 0x51544B52u;  // 'QTKR'
constexpr uint32_t kTokVersion = 1;
constexpr uint32_t kTokMaxVocab = 1000000;
constexpr uint32_t kTokMaxMerges = 1000000;
constexpr size_t kTokMaxText = 1024 * 1024;
constexpr uint32_t kDead = UINT32_MAX;  // a merged-away slot

bool read_u32(FILE* f, uint32_t* v) {
    uint8_t b[4];
    if (std::fread(b, 1, 4, f) != 4) return false;
    *v = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
    return true;
}

void release(q_tokenizer* tok) {
    if (tok->vocab) {
        for (uint32_t i = 0; i < tok->vocab_size; ++i) std::free(tok->vocab[i]);
        std::free(static_cast<void*>(tok->vocab));
        tok->vocab = nullptr;
    }
    std::free(tok->merges);
    tok->merges = nullptr;
    delete tok->merge_hash_table;
    tok->merge_hash_table = nullptr;
}

q_error_code build_table(q_tokenizer* tok) {
    bpe_hash_table* t = new (std::nothrow) bpe_hash_table();
    if (!t) return Q_ERR_ALLOC_FAILED;
    try {
        std::unordered_map<uint64_t, uint32_t> last;  // key -> last rule of that key
        last.reserve((size_t)tok->num_merges * 2);
        for (uint32_t i = 0; i < tok->num_merges; ++i) {
            const q_bpe_merge& m = tok->merges[i];
            last[((uint64_t)m.token_id1 << 16) | m.token_id2] = i;
        }
        t->merged.resize(tok->num_merges);
        for (uint32_t i = 0; i < tok->num_merges; ++i) {
            const q_bpe_merge& m = tok->merges[i];
            t->merged[i] = tok->merges[last[((uint64_t)m.token_id1 << 16) | m.token_id2]].merged_id;
        }
    } catch (const std::bad_alloc&) {
        delete t;
        return Q_ERR_ALLOC_FAILED;
    }
    tok->merge_hash_table = t;
    return Q_OK;
}

// The greedy merge passes over ids[0..n), in place; returns the live count.
size_t apply_merges(const q_tokenizer* tok, uint32_t* ids, size_t n) {
    if (tok->num_merges == 0 || n < 2) return n;
    const bpe_hash_table* table = tok->merge_hash_table;
    // Live-token counts: a rule whose ids are absent cannot match, so its
    // scan is skipped (the result is that of scanning).
    std::unordered_map<uint32_t, uint32_t> count;
    for (size_t j = 0; j < n; ++j) ++count[ids[j]];
    auto present = [&](uint32_t id) {
        auto it = count.find(id);
        return it != count.end() && it->second != 0;
    };
    bool changed = true;
    while (changed) {
        changed = false;
        for (uint32_t r = 0; r < tok->num_merges; ++r) {
            const uint32_t a = tok->merges[r].token_id1, b = tok->merges[r].token_id2;
            if (!present(a) || !present(b) || (a == b && count[a] < 2)) continue;
            const uint32_t m = table ? table->merged[r] : tok->merges[r].merged_id;
            for (size_t j = 0; j < n; ++j) {
                if (ids[j] == kDead) continue;
                size_t k = j + 1;
                while (k < n && ids[k] == kDead) ++k;
                if (k >= n) break;
                if (ids[j] == a && ids[k] == b) {
                    ids[j] = m;
                    ids[k] = kDead;
                    --count[a];
                    --count[b];
                    ++count[m];
                    changed = true;
                }
            }
        }
        // drop the dead slots before the next pass
        size_t w = 0;
        for (size_t j = 0; j < n; ++j)
            if (ids[j] != kDead) ids[w++] = ids[j];
        n = w;
    }
    return n;
}

}  // namespace

extern "C" {

// Reference src/tokenizer/bpe.c:263-... (load): NULL tok or path ->
// INVALID_ARG; the struct is zeroed; unopenable file or a short read ->
// FILE_OPEN; bad magic -> INVALID_MAGIC; version != 1 -> INVALID_ARG;
// vocab_size 0 or above 1e6, or more than 1e6 merges -> INVALID_SIZE; an
// empty vocab entry -> INVALID_SIZE; a merge id outside the vocabulary ->
// INVALID_ARG.  On failure the vocabulary and merges read so far are freed
// (and their pointers cleared).
q_error_code q_tokenizer_load(q_tokenizer* __restrict__ tok, const char* tokenizer_path) {
    if (!tok || !tokenizer_path) return Q_ERR_INVALID_ARG;
    std::memset(tok, 0, sizeof(*tok));
    FILE* f = std::fopen(tokenizer_path, "rb");
    if (!f) return Q_ERR_FILE_OPEN;
    q_error_code rc = Q_OK;
    uint32_t magic = 0, version = 0, n_merges = 0, reserved = 0;
    auto fail = [&](q_error_code c) {
        release(tok);
        std::fclose(f);
        return c;
    };
    if (!read_u32(f, &magic)) return fail(Q_ERR_FILE_OPEN);
    if (magic != kTokMagic) return fail(Q_ERR_INVALID_MAGIC);
    if (!read_u32(f, &version)) return fail(Q_ERR_FILE_OPEN);
    if (version != kTokVersion) return fail(Q_ERR_INVALID_ARG);
    if (!read_u32(f, &tok->vocab_size) || !read_u32(f, &n_merges) || !read_u32(f, &tok->bos_token_id) ||
        !read_u32(f, &tok->eos_token_id) || !read_u32(f, &tok->pad_token_id) || !read_u32(f, &reserved))
        return fail(Q_ERR_FILE_OPEN);
    if (tok->vocab_size == 0 || tok->vocab_size > kTokMaxVocab) return fail(Q_ERR_INVALID_SIZE);
    if (n_merges > kTokMaxMerges) return fail(Q_ERR_INVALID_SIZE);
    tok->vocab = static_cast<char**>(std::calloc(tok->vocab_size, sizeof(char*)));
    if (!tok->vocab) return fail(Q_ERR_ALLOC_FAILED);
    for (uint32_t i = 0; i < tok->vocab_size; ++i) {
        uint8_t len = 0;
        if (std::fread(&len, 1, 1, f) != 1) return fail(Q_ERR_FILE_OPEN);
        if (len == 0) return fail(Q_ERR_INVALID_SIZE);
        char* s = static_cast<char*>(std::malloc((size_t)len + 1));
        if (!s) return fail(Q_ERR_ALLOC_FAILED);
        tok->vocab[i] = s;
        if (std::fread(s, 1, len, f) != len) return fail(Q_ERR_FILE_OPEN);
        s[len] = '\0';
    }
    tok->num_merges = n_merges;
    if (n_merges > 0) {
        tok->merges = static_cast<q_bpe_merge*>(std::calloc(n_merges, sizeof(q_bpe_merge)));
        if (!tok->merges) return fail(Q_ERR_ALLOC_FAILED);
        for (uint32_t i = 0; i < n_merges; ++i) {
            q_bpe_merge& m = tok->merges[i];
            if (!read_u32(f, &m.token_id1) || !read_u32(f, &m.token_id2) || !read_u32(f, &m.merged_id))
                return fail(Q_ERR_FILE_OPEN);
            if (m.token_id1 >= tok->vocab_size || m.token_id2 >= tok->vocab_size || m.merged_id >= tok->vocab_size)
                return fail(Q_ERR_INVALID_ARG);
        }
        if ((rc = build_table(tok)) != Q_OK) return fail(rc);
    }
    std::fclose(f);
    tok->initialized = true;
    return Q_OK;
}

// Reference src/tokenizer/bpe.c:692-808 (encode): NULL tok, text, tokens_out
// or num_tokens_out, or a tokenizer not initialized -> INVALID_ARG;
// max_tokens 0 -> INVALID_SIZE; empty text -> only BOS/EOS as requested
// (ARENA_OOM when they do not fit); text longer than 1 MiB -> ARENA_OOM;
// the final token count above max_tokens -> ARENA_OOM (nothing written).
q_error_code q_tokenizer_encode(q_tokenizer* __restrict__ tok, const char* __restrict__ text,
                                uint32_t* __restrict__ tokens_out, uint32_t* __restrict__ num_tokens_out,
                                uint32_t max_tokens, bool add_bos, bool add_eos) {
    if (!tok || !text || !tokens_out || !num_tokens_out || !tok->initialized) return Q_ERR_INVALID_ARG;
    if (max_tokens == 0) return Q_ERR_INVALID_SIZE;
    if (text[0] == '\0') {
        *num_tokens_out = 0;
        const uint32_t need = (add_bos ? 1u : 0u) + (add_eos ? 1u : 0u);
        if (need == 0) return Q_OK;
        if (need > max_tokens) return Q_ERR_ARENA_OOM;
        uint32_t n = 0;
        if (add_bos) tokens_out[n++] = tok->bos_token_id;
        if (add_eos) tokens_out[n++] = tok->eos_token_id;
        *num_tokens_out = n;
        return Q_OK;
    }
    const size_t len = std::strlen(text);
    if (len > kTokMaxText) return Q_ERR_ARENA_OOM;
    std::vector<uint32_t> ids;
    try {
        ids.resize(len + 2);
    } catch (const std::bad_alloc&) {
        return Q_ERR_ALLOC_FAILED;
    }
    for (size_t i = 0; i < len; ++i) {
        const uint32_t b = (uint8_t)text[i];
        ids[i + 1] = b < tok->vocab_size ? b : tok->pad_token_id;
    }
    size_t n = 0;
    try {
        n = apply_merges(tok, ids.data() + 1, len);
    } catch (const std::bad_alloc&) {
        return Q_ERR_ALLOC_FAILED;
    }
    const uint32_t* first = ids.data() + 1;
    if (add_bos) {
        ids[0] = tok->bos_token_id;
        first = ids.data();
        ++n;
    }
    if (add_eos) ids[(add_bos ? 0 : 1) + n++] = tok->eos_token_id;
    if (n > (size_t)max_tokens) return Q_ERR_ARENA_OOM;
    std::memcpy(tokens_out, first, n * sizeof(uint32_t));
    *num_tokens_out = (uint32_t)n;
    return Q_OK;
}

// Reference src/tokenizer/bpe.c:811-866 (decode): NULL tok, tokens or
// text_out, or a tokenizer not initialized -> INVALID_ARG; text_buf_size 0
// -> INVALID_SIZE.  BOS, EOS and pad ids and ids outside the vocabulary are
// skipped; each token adds its string up to its first NUL.  A token whose
// string would reach the buffer's last two bytes ends the text there with
// ARENA_OOM (the reference's bound: pos + len >= size - 1).
q_error_code q_tokenizer_decode(q_tokenizer* __restrict__ tok, const uint32_t* __restrict__ tokens,
                                uint32_t num_tokens, char* __restrict__ text_out, size_t text_buf_size) {
    if (!tok || !tokens || !text_out || !tok->initialized) return Q_ERR_INVALID_ARG;
    if (text_buf_size == 0) return Q_ERR_INVALID_SIZE;
    size_t pos = 0;
    for (uint32_t i = 0; i < num_tokens; ++i) {
        const uint32_t id = tokens[i];
        if (id == tok->bos_token_id || id == tok->eos_token_id || id == tok->pad_token_id) continue;
        if (id >= tok->vocab_size || !tok->vocab || !tok->vocab[id]) continue;
        const char* s = tok->vocab[id];
        const size_t l = std::strlen(s);
        if (pos + l >= text_buf_size - 1) {
            text_out[pos] = '\0';
            return Q_ERR_ARENA_OOM;
        }
        std::memcpy(text_out + pos, s, l);
        pos += l;
    }
    text_out[pos] = '\0';
    return Q_OK;
}

// Reference src/tokenizer/bpe.c:869-887: frees the vocabulary strings, the
// merges and the table, and zeroes the struct; NULL is a no-op.
void q_tokenizer_free(q_tokenizer* __restrict__ tok) {
    if (!tok) return;
    release(tok);
    std::memset(tok, 0, sizeof(*tok));
}

}  // extern "C"
