"""q_generate's validation order and codes (reference src/main.c:994-1026),
checked without a GPU: every case fails before the first forward pass."""
import ctypes as C

import numpy as np

import qorus_amd as qa


def state(**kw):
    ctx, model, tok = qa.QContext(), qa.QLlamaModel(), qa.QTokenizer()
    prompt = np.array([1, 2, 3], np.uint32)
    out = np.zeros(8, np.uint32)
    keep = [ctx, model, tok, prompt, out]
    tok.initialized = True
    model.config.vocab_size = 100
    model.config.max_seq_len = 16
    ctx.scratch_buffer = prompt.ctypes.data   # non-NULL stand-ins: never dereferenced by validation
    ctx.kv_buffer = prompt.ctypes.data
    st = qa.QGenerationState(C.addressof(ctx), C.addressof(model), C.addressof(tok), prompt.ctypes.data, 3,
                             out.ctypes.data, 0, 8, 0.5, 0, 0.0, 0)
    for k, v in kw.items():
        if k in ("initialized",):
            tok.initialized = v
        elif k in ("scratch_buffer", "kv_buffer"):
            setattr(ctx, k, v)
        elif k == "max_seq_len":
            model.config.max_seq_len = v
        else:
            setattr(st, k, v)
    return st, keep


def test_q_generate_validation_codes():
    lib = qa.lib()
    g = lambda st: lib.q_generate(C.byref(st))
    assert lib.q_generate(None) == -10
    for field in ("ctx", "model", "tokenizer", "prompt_tokens", "generated_tokens"):
        st, keep = state(**{field: None})
        assert g(st) == -10, field
    st, keep = state(num_prompt_tokens=0)
    assert g(st) == -15
    st, keep = state(max_tokens=0)
    assert g(st) == -15
    for t in (-1.0, float("nan"), float("inf")):
        st, keep = state(temperature=t)
        assert g(st) == -10, t
    st, keep = state(initialized=False)
    assert g(st) == -10
    st, keep = state(scratch_buffer=None)
    assert g(st) == -10
    st, keep = state(kv_buffer=None)
    assert g(st) == -10
    st, keep = state(max_seq_len=2)  # 3 prompt tokens > max_seq_len
    assert g(st) == -15
    # the order: a zero max_tokens is reported before a bad temperature
    st, keep = state(max_tokens=0, temperature=-1.0)
    assert g(st) == -15
