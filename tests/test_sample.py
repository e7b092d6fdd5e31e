"""Sampling: q_sample_token with temperature, top-k and top-p.

The oracle's restatement (or_sample_token) is checked token for token
against the reference's own sampler (oracle/_ref: src/main.c compiled from
its sources, arena path, each test on a private copy of the library so its
thread-local xorshift64* state starts at 123456789), on inputs whose
top-k/top-p cut has no ties between nonzero probabilities.  The device
sampler (this build's q_sample_token) is checked token for token against
the oracle, with the RNG state synchronised through qh_sample_set_state,
up to the Llama-3 vocabulary (128256) where the reference itself takes
seconds (top-k: quadratic quickselect over the exactly-zero probabilities
of its clamped polynomial exp) or overflows its stack (top-p: recursive
quicksort).  Bar: identical tokens (integer output) and an identical RNG
stream.  The reference's property tests (tests/test_main.c) run on both.
"""
import ctypes as C

import numpy as np
import pytest

import qorus_amd as qa
from qorus_amd import _lib as L
from oracle import oracle as orc

needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built (needs /root/reference)")

FILTERS = [(5, 0.0), (40, 0.0), (0, 0.5), (0, 0.9), (10, 0.8), (0, 1.0), ("V", 0.0), ("V+5", 0.3)]


def logits_for(V, rng, scale=1.0, aligned=True, ties=False):
    """float32 logits; aligned: 32-byte aligned data (the reference's vector
    temperature path), else offset by one float; ties: rounded to halves."""
    x = rng.standard_normal(V).astype(np.float32) * np.float32(scale)
    if ties:
        x = (np.round(x * 2) / 2).astype(np.float32)
    buf = orc.aligned_empty((V + 8,), np.float32, 64)
    off = 0 if aligned else 1
    out = buf[off:off + V]
    out[:] = x
    assert (out.ctypes.data % 32 == 0) == aligned
    return out


def k_of(k, V):
    return V if k == "V" else (V + 5 if k == "V+5" else k)


def ref_cases():
    for V in (8, 16, 64, 100, 1000, 4096):
        for T in (0.5, 1.0, 1.7):
            for k, p in FILTERS:
                yield V, T, k_of(k, V), p


# ---------------------------------------------------------------- CPU ----

@needs_ref
def test_oracle_sampler_matches_reference(tmp_path):
    R = orc.RefSampler(tmp_path)
    state = C.c_uint64(orc.RNG_SEED)
    rng = np.random.default_rng(2024)
    n = 0
    try:
        for V, T, k, p in ref_cases():
            for aligned in (True, False):
                lg = logits_for(V, rng, scale=1.0, aligned=aligned)
                rc, t_ref = R.sample(lg, T, k, p)
                assert rc == 0
                t_or = orc.sample_token(lg, T, k, p, state)
                assert t_or == t_ref, (V, T, k, p, aligned)
                n += 1
    finally:
        R.close()
    assert n == 288


def test_reference_property_tests_on_oracle():
    """tests/test_main.c (reference): valid token, top-k membership, nucleus
    membership, greedy argmax."""
    state = C.c_uint64(orc.RNG_SEED)
    lg = orc.aligned_copy(np.arange(100, dtype=np.float32) / np.float32(10))
    assert 0 <= orc.sample_token(lg, 1.0, 0, 0.0, state) < 100
    lg = orc.aligned_copy((100 - np.arange(100)).astype(np.float32))
    for _ in range(10):
        assert orc.sample_token(lg, 1.0, 10, 0.0, state) < 10
    lg = orc.aligned_copy((50 - 2 * np.arange(50)).astype(np.float32))
    nucleus = nucleus_of_test_main(lg, 0.9)
    for _ in range(10):
        assert orc.sample_token(lg, 1.0, 0, 0.9, state) in nucleus


def nucleus_of_test_main(lg, top_p):
    """The nucleus as tests/test_main.c:204-243 computes it (libm softmax,
    descending sort, first prefix reaching top_p)."""
    e = np.exp(lg.astype(np.float64) - lg.max())
    pr = e / e.sum()
    order = np.argsort(-pr, kind="stable")
    c = np.cumsum(pr[order])
    n = int(np.searchsorted(c, top_p) + 1)
    return set(order[:n].tolist())


def test_sample_validation_without_device():
    """Reference main.c:862-866 validation order and codes; decided before
    any device work."""
    lib = qa.lib()
    lg = orc.aligned_copy(np.zeros(10, np.float32))
    tok = C.c_uint32()
    p = lg.ctypes.data
    assert lib.q_sample_token(None, 10, 1.0, 0, 0.0, C.byref(tok), None) == L.Q_ERR_INVALID_ARG
    assert lib.q_sample_token(p, 10, 1.0, 0, 0.0, None, None) == L.Q_ERR_INVALID_ARG
    assert lib.q_sample_token(p, 0, 1.0, 0, 0.0, C.byref(tok), None) == L.Q_ERR_INVALID_SIZE
    assert lib.q_sample_token(p, 10, -1.0, 0, 0.0, C.byref(tok), None) == L.Q_ERR_INVALID_ARG
    assert lib.q_sample_token(p, 10, float("nan"), 0, 0.0, C.byref(tok), None) == L.Q_ERR_INVALID_ARG
    assert lib.q_sample_token(p, 10, float("inf"), 0, 0.0, C.byref(tok), None) == L.Q_ERR_INVALID_ARG


def arena_ctx(lib, nbytes):
    ctx = orc.QContext()
    assert lib.q_alloc_arena(C.byref(ctx), nbytes) == 0
    return ctx


@needs_ref
@pytest.mark.parametrize("arena", [2048, 5000, 6000, 9000, 13000, 17100])
def test_sample_arena_oom_matches_reference(tmp_path, arena):
    """Where the reference runs out of arena (main.c:891-899, 451-454,
    740-743), this build returns the same code with the arena at the same
    offset; the RNG does not advance on those paths."""
    V, T, k, p = 1000, 1.0, 10, 0.9
    lg = logits_for(V, np.random.default_rng(5))
    R = orc.RefSampler(tmp_path, arena_bytes=arena)
    lib = qa.lib()
    ctx = arena_ctx(lib, arena)
    try:
        rc_ref, _ = R.sample(lg, T, k, p)
        if rc_ref != L.Q_ERR_ARENA_OOM:
            pytest.skip("the reference does not run out of arena here (covered on the GPU)")
        s0 = lib.qh_sample_get_state()
        tok = C.c_uint32()
        rc = lib.q_sample_token(lg.ctypes.data, V, T, k, p, C.byref(tok), C.byref(ctx))
        assert rc == rc_ref
        assert ctx.scratch_head == R.ctx.scratch_head
        assert lib.qh_sample_get_state() == s0
    finally:
        R.close()
        lib.q_free_memory(C.byref(ctx))


# ---------------------------------------------------------------- GPU ----

def device_sample(lib, lg, T, k, p, ctx=None):
    tok = C.c_uint32(0xFFFFFFFF)
    rc = lib.q_sample_token(lg.ctypes.data, lg.size, T, k, p, C.byref(tok), C.byref(ctx) if ctx else None)
    assert rc == 0, lib.qh_last_error().decode()
    return tok.value


def device_cases():
    for V in (8, 16, 64, 1000, 4096, 32000, 128256):
        for T in (0.6, 1.0, 1.5):
            for k, p in FILTERS + [(0, 0.0), (1, 0.0), (1000, 0.0), (50, 0.9), (0, 0.95)]:
                yield V, T, k_of(k, V), p


@pytest.mark.gpu
def test_device_sampler_matches_oracle():
    lib = qa.lib()
    seed = 987654321
    lib.qh_sample_set_state(seed)
    state = C.c_uint64(seed)
    rng = np.random.default_rng(77)
    n = 0
    for V, T, k, p in device_cases():
        for aligned, ties, scale in ((True, False, 1.0), (False, False, 1.0), (True, True, 1.0), (True, False, 0.05)):
            lg = logits_for(V, rng, scale=scale, aligned=aligned, ties=ties)
            t_dev = device_sample(lib, lg, T, k, p)
            t_or = orc.sample_token(lg, T, k, p, state)
            assert t_dev == t_or, (V, T, k, p, aligned, ties, scale)
            n += 1
    assert lib.qh_sample_get_state() == state.value
    print(f"{n} sampled tokens identical")


@pytest.mark.gpu
def test_device_sampler_small_vocab():
    """V < 8: the sampler's scalar softmax (libm expf) on inputs whose
    exponentials are exact (0 and far-below-max differences)."""
    lib = qa.lib()
    lib.qh_sample_set_state(42)
    state = C.c_uint64(42)
    lg = orc.aligned_copy(np.array([0, 0, -200, 0, -200], np.float32))
    for k, p in ((0, 0.0), (2, 0.0), (0, 0.5), (0, 1.0), (5, 0.0)):
        for _ in range(4):
            assert device_sample(lib, lg, 1.0, k, p) == orc.sample_token(lg, 1.0, k, p, state)


@pytest.mark.gpu
@needs_ref
def test_device_sampler_matches_reference(tmp_path):
    """The device sampler against the reference binary itself, lockstep RNG
    (both start at 123456789)."""
    lib = qa.lib()
    lib.qh_sample_set_state(orc.RNG_SEED)
    R = orc.RefSampler(tmp_path)
    rng = np.random.default_rng(31)
    try:
        for V, T, k, p in ref_cases():
            lg = logits_for(V, rng)
            rc, t_ref = R.sample(lg, T, k, p)
            assert rc == 0
            assert device_sample(lib, lg, T, k, p) == t_ref, (V, T, k, p)
    finally:
        R.close()


@pytest.mark.gpu
def test_device_reference_property_tests():
    """tests/test_main.c (reference) on the device sampler."""
    lib = qa.lib()
    lg = orc.aligned_copy(np.arange(100, dtype=np.float32) / np.float32(10))
    assert device_sample(lib, lg, 1.0, 0, 0.0) < 100
    lg = orc.aligned_copy((50 - np.abs(np.arange(50) - 25)).astype(np.float32))
    s0 = lib.qh_sample_get_state()
    for _ in range(5):
        assert device_sample(lib, lg, 0.0, 0, 0.0) == 25  # greedy
    assert lib.qh_sample_get_state() == s0  # greedy draws nothing
    lg = orc.aligned_copy((100 - np.arange(100)).astype(np.float32))
    for _ in range(10):
        assert device_sample(lib, lg, 1.0, 10, 0.0) < 10
    lg = orc.aligned_copy((50 - 2 * np.arange(50)).astype(np.float32))
    nucleus = nucleus_of_test_main(lg, 0.9)
    for _ in range(10):
        assert device_sample(lib, lg, 1.0, 0, 0.9) in nucleus
    lg = orc.aligned_copy((20 - np.arange(20)).astype(np.float32))
    for T in (0.5, 1.0, 2.0):
        assert device_sample(lib, lg, T, 0, 0.0) < 20


@pytest.mark.gpu
@needs_ref
@pytest.mark.parametrize("arena", [9000, 13000, 17100, 23000, 1 << 20])
def test_device_sampler_arena_matches_reference(tmp_path, arena):
    """Arena-backed calls: same code, same arena offset and the same token,
    including 23000 bytes, where only the reference's top-p prefix-sum
    buffer does not fit (its nucleus then keeps every token)."""
    V, T, k, p = 1000, 1.0, 10, 0.9
    lib = qa.lib()
    lib.qh_sample_set_state(orc.RNG_SEED)
    R = orc.RefSampler(tmp_path, arena_bytes=arena)
    ctx = arena_ctx(lib, arena)
    rng = np.random.default_rng(arena)
    try:
        for _ in range(3):
            lg = logits_for(V, rng)
            lib.q_arena_reset(C.byref(ctx))
            rc_ref, t_ref = R.sample(lg, T, k, p)
            tok = C.c_uint32()
            rc = lib.q_sample_token(lg.ctypes.data, V, T, k, p, C.byref(tok), C.byref(ctx))
            assert rc == rc_ref
            assert ctx.scratch_head == R.ctx.scratch_head
            if rc == 0:
                assert tok.value == t_ref
    finally:
        R.close()
        lib.q_free_memory(C.byref(ctx))
