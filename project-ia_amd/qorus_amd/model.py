"""Python handle over the reference model API of libqorus_hip.so:
q_init_memory -> q_alloc_kv_cache -> q_alloc_arena -> llama_build_graph ->
llama_forward / qh_llama_generate -> llama_free_graph -> q_free_memory."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib
from .model_file import QorusHeader


class QContext(C.Structure):
    """q_context (reference include/qorus_types.h:215-231), 72 bytes."""
    _fields_ = [("weights_mmap", C.c_void_p), ("weights_size", C.c_size_t), ("header", C.c_void_p),
                ("kv_buffer", C.c_void_p), ("kv_size", C.c_size_t),
                ("scratch_buffer", C.c_void_p), ("scratch_size", C.c_size_t),
                ("scratch_head", C.c_size_t), ("scratch_base_offset", C.c_size_t)]


class QLlamaConfig(C.Structure):
    _fields_ = [("vocab_size", C.c_uint32), ("dim", C.c_uint32), ("hidden_dim", C.c_uint32),
                ("n_layers", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("max_seq_len", C.c_uint32), ("rope_freq_base", C.c_float), ("rms_norm_eps", C.c_float)]


class QLlamaModel(C.Structure):
    """q_llama_model (reference include/qorus_types.h:265-286)."""
    _fields_ = [("config", QLlamaConfig), ("token_embd", C.c_void_p), ("output_norm", C.c_void_p),
                ("output", C.c_void_p), ("layers", C.c_void_p), ("rope_freqs", C.c_void_p),
                ("rope_cache_enabled", C.c_bool), ("rope_cos_cache", C.c_void_p),
                ("rope_sin_cache", C.c_void_p), ("ctx", C.c_void_p)]


assert C.sizeof(QContext) == 72 and C.sizeof(QLlamaModel) == 112


class QGenerationState(C.Structure):
    """q_generation_state (include/qorus_types.h)."""
    _fields_ = [("ctx", C.c_void_p), ("model", C.c_void_p), ("tokenizer", C.c_void_p),
                ("prompt_tokens", C.c_void_p), ("num_prompt_tokens", C.c_uint32),
                ("generated_tokens", C.c_void_p), ("num_generated_tokens", C.c_uint32),
                ("max_tokens", C.c_uint32), ("temperature", C.c_float), ("top_k", C.c_uint32),
                ("top_p", C.c_float), ("current_pos", C.c_uint32)]


class Model:
    """A loaded v3 model with an HBM KV cache sized for its max_seq_len."""

    def __init__(self, path: str):
        L = lib()
        self.ctx = QContext()
        self.model = QLlamaModel()
        self._closed = False
        check(L.q_init_memory(C.byref(self.ctx), str(path).encode()), "q_init_memory")
        h = QorusHeader(*C.cast(self.ctx.header, C.POINTER(C.c_uint32 * 9)).contents[2:9])
        self.head_dim = h.dim // h.n_heads
        self.kv_floats_per_layer = h.n_kv * h.max_seq * 2 * self.head_dim
        kv_bytes = h.n_layers * self.kv_floats_per_layer * 4
        check(L.q_alloc_kv_cache(C.byref(self.ctx), kv_bytes), "q_alloc_kv_cache")
        arena = (1 << 24) + 2 * h.max_seq * self.head_dim * 4 + 64 * 1024 * (1 + h.n_layers)
        check(L.q_alloc_arena(C.byref(self.ctx), arena), "q_alloc_arena")
        check(L.llama_build_graph(C.byref(self.ctx), C.byref(self.model)), "llama_build_graph")
        c = self.model.config
        self.vocab, self.dim, self.n_layers = c.vocab_size, c.dim, c.n_layers
        self.n_kv, self.max_seq = c.n_kv_heads, c.max_seq_len

    def upload_kv(self, kv: np.ndarray):
        """Write the whole cache [L][n_kv][max_seq][2][head_dim] (float32)."""
        kv = np.ascontiguousarray(kv, dtype=np.float32)
        assert kv.size == self.n_layers * self.kv_floats_per_layer
        check(lib().qh_memcpy_htod(self.ctx.kv_buffer, kv.ctypes.data, kv.nbytes), "kv upload")

    def download_kv(self) -> np.ndarray:
        out = np.empty(self.n_layers * self.kv_floats_per_layer, dtype=np.float32)
        check(lib().qh_memcpy_dtoh(out.ctypes.data, self.ctx.kv_buffer, out.nbytes), "kv download")
        return out

    def forward(self, tokens, pos: int) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.vocab, dtype=np.float32)
        check(lib().llama_forward(C.byref(self.model), C.byref(self.ctx), toks.ctypes.data, toks.size, pos,
                                  logits.ctypes.data), "llama_forward")
        return logits

    def generate(self, token: int, pos: int, n: int):
        out = np.empty(n, dtype=np.uint32)
        ms = C.c_float()
        check(lib().qh_llama_generate(C.byref(self.model), C.byref(self.ctx), token, pos, n, out.ctypes.data,
                                      C.byref(ms)), "qh_llama_generate")
        return out, float(ms.value)

    def generate_sampled(self, token: int, pos: int, n: int, temperature: float, top_k: int = 0,
                         top_p: float = 0.0):
        """qh_llama_generate_sampled: n device steps, each token sampled on
        the device (q_sample_token semantics, this thread's RNG stream)."""
        out = np.empty(n, dtype=np.uint32)
        ms = C.c_float()
        check(lib().qh_llama_generate_sampled(C.byref(self.model), C.byref(self.ctx), token, pos, n, temperature,
                                              top_k, top_p, out.ctypes.data, C.byref(ms)),
              "qh_llama_generate_sampled")
        return out, float(ms.value)

    def q_generate(self, tokenizer, prompt, max_tokens: int, temperature: float = 0.0, top_k: int = 0,
                   top_p: float = 0.0):
        """q_generate from position 0: returns (generated token ids,
        current_pos); raises QorusError on a failing code."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        st = QGenerationState(C.addressof(self.ctx), C.addressof(self.model), C.addressof(tokenizer.t),
                              p.ctypes.data, p.size, out.ctypes.data, 0, max_tokens, temperature, top_k, top_p, 0)
        check(lib().q_generate(C.byref(st)), "q_generate")
        return out[:st.num_generated_tokens].tolist(), st.current_pos

    def close(self):
        if not self._closed:
            lib().llama_free_graph(C.byref(self.model))
            lib().q_free_memory(C.byref(self.ctx))
            self._closed = True

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
