"""GPU parity of the batched prefill: llama_forward with seq_len > 1 (every
projection on the MFMA GEMM with the RMSNorm / SwiGLU product made where it
converts its rows, RoPE + KV-cache stores, causal attention of the prompt's
queries over the cache on matrix cores, chunks of up to 2048 tokens)
against the oracle's token-by-token decode steps (or_decode_step), which is
what the prefill must equal: token t of the prompt attends the cached keys
0 .. pos + t.

Bars (the decode step's, written out):
  * logits of the last token: max |gpu - oracle| <= 1e-4 * max |oracle logit|;
  * greedy token equal;
  * every KV-cache row the prompt writes: max |gpu - oracle| <= 1e-4 * max |row|
    per layer; rows outside the prompt keep their bits;
  * decode steps after the prefill (reading the prefilled rows) give the
    oracle's greedy tokens.
"""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def build(qa, tmp_path, h, seed, prefill, name="m.qorus"):
    path = tmp_path / name
    qa.synthetic.write_synthetic_model(path, h, seed)
    m = qa.Model(path)
    hd = h.dim // h.n_heads
    rng = orc.rng_for(seed, 99)
    kv = np.zeros((h.n_layers, h.n_kv, h.max_seq, 2, hd), np.float32)
    kv[:, :, :prefill] = rng.standard_normal((h.n_layers, h.n_kv, prefill, 2, hd), dtype=np.float32)
    m.upload_kv(kv)
    blob = np.fromfile(path, dtype=np.uint8)
    return m, blob, kv


def rel_err(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))


def oracle_prompt(ref, toks, pos):
    for i, t in enumerate(toks[:-1]):
        ref.fill(t, pos + i)
    return ref.step(toks[-1], pos + len(toks) - 1)


def check_prompt(qa, m, h, kv0, ref, toks, pos, label=""):
    print(f"prefill {label}: T={len(toks)} pos={pos}", flush=True)
    lg = m.forward(toks, pos)
    tok_ref, lg_ref = oracle_prompt(ref, toks, pos)
    e = rel_err(lg, lg_ref)
    print(f"  logits rel err {e:.3e}", flush=True)
    assert e <= 1e-4, (label, e)
    assert int(np.argmax(lg)) == tok_ref, label
    kv_gpu = m.download_kv().reshape(kv0.shape)
    T = len(toks)
    for l in range(h.n_layers):
        got = kv_gpu[l, :, pos:pos + T]
        want = ref.kv[l, :, pos:pos + T]
        ek = rel_err(got, want)
        assert ek <= 1e-4, (label, l, ek)
    # rows outside the prompt keep their bits
    assert np.array_equal(kv_gpu[:, :, :pos], kv0[:, :, :pos])
    assert np.array_equal(kv_gpu[:, :, pos + T:], kv0[:, :, pos + T:])
    return tok_ref


@pytest.mark.parametrize("n_heads,n_kv", [(4, 1), (8, 1), (16, 2), (2, 2), (8, 2)])
def test_prefill_gqa_groups(qa, tmp_path, n_heads, n_kv):
    """GQA groups 4, 8, 8, 1 and 4 (the attention kernel is instantiated per
    group); a 37-token prompt at position 0 (query tiles of 16: the last one
    ragged; rows of fewer than 8 keys use the reference's libm exp)."""
    h = qa.QorusHeader(vocab=700, dim=128 * n_heads, hidden=1024, n_layers=2, n_heads=n_heads, n_kv=n_kv,
                       max_seq=128)
    m, blob, kv = build(qa, tmp_path, h, 31 + n_heads + n_kv, 0)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        rng = orc.rng_for(n_heads, n_kv)
        toks = [int(t) for t in rng.integers(0, h.vocab, 37)]
        check_prompt(qa, m, h, kv, ref, toks, 0, f"group {n_heads // n_kv}")
    finally:
        m.close()


def test_prefill_continues_a_cached_context(qa, tmp_path):
    """A 20-token prompt at position 50 over a random cache: its queries
    attend the 50 cached keys too (the reference's own seq_len > 1 branch
    would not); then greedy decode steps read the prefilled rows."""
    h = qa.QorusHeader(vocab=500, dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv=2, max_seq=128)
    P = 50
    m, blob, kv = build(qa, tmp_path, h, 41, P)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(41, 1).integers(0, h.vocab, 20)]
        tok = check_prompt(qa, m, h, kv, ref, toks, P)
        n = 6
        got, _ = m.generate(tok, P + 20, n)
        want, t = [], tok
        for i in range(n):
            t, _ = ref.step(t, P + 20 + i)
            want.append(t)
        assert got.tolist() == want
    finally:
        m.close()


@pytest.mark.parametrize("T", [2, 8, 9, 16, 17])
def test_prefill_short_prompts(qa, tmp_path, T):
    """Prompts of 2 to 17 tokens at position 0: query rows with fewer than 8
    keys (libm exp, divided by the sum), exactly 8, the first polynomial
    row, one full and one ragged 16-query tile."""
    h = qa.QorusHeader(vocab=300, dim=256, hidden=512, n_layers=3, n_heads=2, n_kv=1, max_seq=64)
    m, blob, kv = build(qa, tmp_path, h, 50 + T, 0)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(50, T).integers(0, h.vocab, T)]
        check_prompt(qa, m, h, kv, ref, toks, 0, f"T={T}")
    finally:
        m.close()


@pytest.mark.parametrize("T", [5, 33, 100])
def test_prefill_small_tiles_with_k_splits(qa, tmp_path, T):
    """Widths with 32 and 64 blocks per row, so that prompts of 5, 33 and
    100 tokens take the 16-, 64- and 128-token tiles with K splits of 2-4:
    the split-K partials summed by the next row conversion (W_down's, with
    dim <= hidden) and by the RoPE/KV pass (Q|K|V's)."""
    h = qa.QorusHeader(vocab=500, dim=1024, hidden=2048, n_layers=2, n_heads=8, n_kv=2, max_seq=128)
    m, blob, kv = build(qa, tmp_path, h, 70 + T, 0)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(70, T).integers(0, h.vocab, T)]
        check_prompt(qa, m, h, kv, ref, toks, 0, f"T={T}")
    finally:
        m.close()


@pytest.mark.parametrize("T", [600, 2100])
def test_prefill_long_prompts_and_chunks(qa, tmp_path, T):
    """A 600-token prompt at position 3 (one chunk), and a 2100-token one: a
    2048-token chunk, then 52 tokens whose queries attend the first chunk's
    keys from the cache."""
    h = qa.QorusHeader(vocab=400, dim=256, hidden=512, n_layers=2, n_heads=2, n_kv=1, max_seq=T + 40)
    m, blob, kv = build(qa, tmp_path, h, 61, 3)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(61, 2).integers(0, h.vocab, T)]
        check_prompt(qa, m, h, kv, ref, toks, 3, f"{T} tokens")
    finally:
        m.close()


def test_prefill_config4_shapes_two_layers(qa, tmp_path):
    """BASELINE config-4 widths (d 4096, GQA 32/8 x 128, FFN 14336, vocab
    128256, theta 500000) with 2 of the 32 layers: a 40-token prompt at
    position 0 (the Q|K|V launch's three segments, the split-K W_down)."""
    h = qa.QorusHeader(vocab=128256, dim=4096, hidden=14336, n_layers=2, n_heads=32, n_kv=8, max_seq=256)
    m, blob, kv = build(qa, tmp_path, h, 71, 0, name="c4.qorus")
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(71, 3).integers(0, h.vocab, 40)]
        check_prompt(qa, m, h, kv, ref, toks, 0, "config-4 shapes")
    finally:
        m.close()


def test_prefill_unfused_wide_dim(qa, tmp_path):
    """d_model 4352 (the decode's generic GEMV layers; the LM head after the
    prefill takes the separate norm + digits launch), GQA 34/17."""
    h = qa.QorusHeader(vocab=300, dim=4352, hidden=1024, n_layers=2, n_heads=34, n_kv=17, max_seq=64)
    m, blob, kv = build(qa, tmp_path, h, 81, 5, name="wide.qorus")
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(81, 4).integers(0, h.vocab, 10)]
        check_prompt(qa, m, h, kv, ref, toks, 5, "wide")
    finally:
        m.close()


def test_causal_mask_entry_points(qa):
    """q_causal_mask_f32_avx2 (host) and qh_causal_mask_f32 (device) against
    or_causal_mask bit for bit, with the reference's validation codes."""
    import ctypes as C
    lib = qa.lib()
    for n, ld in [(1, 1), (2, 2), (7, 7), (9, 17), (64, 64), (257, 264)]:
        rng = orc.rng_for(n, ld)
        m = rng.standard_normal((n, ld)).astype(np.float32)
        if n > 2:
            m.view(np.uint32)[n - 1, 0] = 0x7FC01234
        want = orc.causal_mask(m, n, -1e9)
        # host form
        h = orc.aligned_copy(m)
        t, keep = orc.make_tensor(h.ctypes.data, (n, n, 1, 1), (ld * 4, 4, 4, 4), orc.Q_F32)
        assert lib.q_causal_mask_f32_avx2(C.addressof(t), -1e9) == 0
        assert np.array_equal(h.view(np.uint32), want.view(np.uint32)), (n, ld)
        # device form
        d = qa.DeviceBuffer.from_numpy(m)
        qa.check(lib.qh_causal_mask_f32(d.ptr, n, ld, -1e9, None))
        qa.check(lib.qh_device_synchronize())
        got = d.download(np.float32, (n, ld))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, ld)
    m = orc.aligned_copy(np.zeros((4, 4), np.float32))
    mk = lambda ne, dt=orc.Q_F32, ptr=m.ctypes.data, ld=4: orc.make_tensor(ptr, (ne[0], ne[1], 1, 1),
                                                                             (ld * 4, 4, 4, 4), dt)
    assert lib.q_causal_mask_f32_avx2(None, -1.0) == -10
    t, k = mk((4, 8))
    assert lib.q_causal_mask_f32_avx2(C.addressof(t), -1.0) == -15
    t, k = mk((0, 0))
    assert lib.q_causal_mask_f32_avx2(C.addressof(t), -1.0) == -15
    t, k = mk((4, 4), orc.Q_Q4_0)
    assert lib.q_causal_mask_f32_avx2(C.addressof(t), -1.0) == -14
    t, k = mk((4, 4), ptr=m.ctypes.data + 4)
    assert lib.q_causal_mask_f32_avx2(C.addressof(t), -1.0) == -13
    t, k = mk((8, 8))
    assert lib.q_causal_mask_f32_avx2(C.addressof(t), -1.0) == -15
    assert lib.qh_causal_mask_f32(None, 4, 4, -1.0, None) == -10
    d = qa.DeviceBuffer(64)
    assert lib.qh_causal_mask_f32(d.ptr, 4, 3, -1.0, None) == -15
    assert lib.qh_causal_mask_f32(d.ptr, 16, 16, -1.0, None) == -10  # 1 KB of rows, a 64-byte buffer


@pytest.mark.parametrize("T", [512, 2048])
def test_prefill_config4_widths(qa, tmp_path, T):
    """The launch plans the bench's 512- and 2048-token prompts time,
    checked: config-4 widths (d 4096, GQA 32/8 x 128, FFN 14336) with 2
    layers and the vocabulary cut to 1024, a T-token prompt at position 0
    (for 512: Q|K|V split-K 2, the 256/192-row cut of W_gate|W_up, W_down
    split 4, register-held scores for 512 keys at GQA group 4; for 2048 the
    two-pass attention over up to 2048 keys), against the oracle's T - 1
    cache fills and last step (spread over host threads; the same bits as
    one).
    W_gate's block scales are divided by 4 (gates of std ~2 instead of ~8):
    the reference's SiLU jumps at g = -10 (its polynomial exp is 91.4 for
    5 < x <= 10 and 22026 above), so a gate within a few ulp of -10 takes
    either side in two correct fp32 orders and moves h_i by ~0.1 |u_i|;
    with the generator's scales 38 of the prompt's 7.3 M layer-0 gates lie
    within 1e-4 of it, and the tokens holding them differed from the oracle
    by up to 1.3e-4 in the next layer's cache rows."""
    import os
    h = qa.QorusHeader(vocab=1024, dim=4096, hidden=14336, n_layers=2, n_heads=32, n_kv=8, max_seq=T + 8)
    path = tmp_path / "c4w.qorus"
    qa.synthetic.write_synthetic_model(path, h, 73)
    blob = np.fromfile(path, dtype=np.uint8)
    lay = qa.model_layout(h)
    for l in range(h.n_layers):
        o = lay[f"{l}.w_gate"]
        g = blob[o: o + h.hidden * (h.dim // 32) * 20].reshape(-1, 20)
        g[:, 16:] = (g[:, 16:].copy().view(np.float32) * np.float32(0.25)).view(np.uint8)
    blob.tofile(path)
    m = qa.Model(path)
    kv = np.zeros((h.n_layers, h.n_kv, h.max_seq, 2, 128), np.float32)
    m.upload_kv(kv)
    orc.set_threads(min(16, os.cpu_count() or 1))
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in orc.rng_for(73, 3).integers(0, h.vocab, T)]
        tok = check_prompt(qa, m, h, kv, ref, toks, 0, f"{T} tokens, config-4 widths")
        # a decode step after the prompt reads the T prefilled rows
        lg = m.forward([tok], T)
        tok_ref, lg_ref = ref.step(tok, T)
        assert rel_err(lg, lg_ref) <= 1e-4
        assert int(np.argmax(lg)) == tok_ref
    finally:
        orc.set_threads(1)
        m.close()


def test_prefill_config4_widths_continued(qa, tmp_path):
    """A 203-token chunk continuing a 1003-key cached context at config-4
    widths (2 layers, vocabulary 1024, W_gate's scales divided by 4 as
    above): every query attends 1004..1206 keys, so the attention takes its
    two-pass form; the steps inside every query of a tile's range take the
    unmasked path from an unaligned first position, and the last query tile
    is partial.  Against the oracle's cache fills and last step."""
    import os
    P, T = 1003, 203
    h = qa.QorusHeader(vocab=1024, dim=4096, hidden=14336, n_layers=2, n_heads=32, n_kv=8, max_seq=P + T + 8)
    path = tmp_path / "c4c.qorus"
    qa.synthetic.write_synthetic_model(path, h, 79)
    blob = np.fromfile(path, dtype=np.uint8)
    lay = qa.model_layout(h)
    for l in range(h.n_layers):
        o = lay[f"{l}.w_gate"]
        g = blob[o: o + h.hidden * (h.dim // 32) * 20].reshape(-1, 20)
        g[:, 16:] = (g[:, 16:].copy().view(np.float32) * np.float32(0.25)).view(np.uint8)
    blob.tofile(path)
    m = qa.Model(path)
    rng = orc.rng_for(79, 5)
    kv = np.zeros((h.n_layers, h.n_kv, h.max_seq, 2, 128), np.float32)
    kv[:, :, :P] = rng.standard_normal((h.n_layers, h.n_kv, P, 2, 128), dtype=np.float32)
    m.upload_kv(kv)
    orc.set_threads(min(16, os.cpu_count() or 1))
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [int(t) for t in rng.integers(0, h.vocab, T)]
        check_prompt(qa, m, h, kv, ref, toks, P, f"{T} tokens at {P}, config-4 widths")
    finally:
        orc.set_threads(1)
        m.close()
