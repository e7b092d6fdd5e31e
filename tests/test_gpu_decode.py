"""GPU parity of the decode step (llama_build_graph / llama_forward /
qh_llama_generate) against the CPU oracle's corrected decode step
(or_decode_step: [out,in] shapes, attention over the KV cache, Q4_0 LM head).

Bars, written out:
  * greedy tokens identical (the north star's decode criterion);
  * logits: max |gpu - oracle| <= 1e-4 * max |oracle logit|;
  * KV cache row written at pos: max |gpu - oracle| <= 1e-4 * max |row|.
The GPU and the oracle differ only in floating-point order (GEMV integer
dots, tree reductions in RMSNorm/softmax/attention sums), see the op tests.
"""
import ctypes as C

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


def test_decode_small_gqa(qa, tmp_path):
    h = qa.QorusHeader(vocab=1000, dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv=1, max_seq=256)
    P = 100
    m, blob, kv = build(qa, tmp_path, h, 11, P)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        tok_ref, lg_ref = ref.step(7, P)
        lg = m.forward([7], P)
        assert rel_err(lg, lg_ref) <= 1e-4
        assert int(np.argmax(lg)) == tok_ref
        kv_gpu = m.download_kv().reshape(kv.shape)
        for l in range(h.n_layers):
            row_ref = ref.kv[l, :, P]
            assert rel_err(kv_gpu[l, :, P], row_ref) <= 1e-4
        # untouched rows stay bit-identical
        assert np.array_equal(kv_gpu[:, :, :P], kv[:, :, :P])
        # greedy generation on the device vs the oracle's greedy loop
        n = 8
        toks, ms = m.generate(tok_ref, P + 1, n)
        want, t = [], tok_ref
        for i in range(n):
            t, _ = ref.step(t, P + 1 + i)
            want.append(t)
        assert toks.tolist() == want
        assert ms > 0
    finally:
        m.close()


@pytest.mark.parametrize("n_heads,n_kv,P", [(8, 1, 130), (16, 2, 63), (2, 2, 200)])
def test_decode_gqa_groups(qa, tmp_path, n_heads, n_kv, P):
    """GQA groups 8 and 1 (the attention kernels are instantiated per group),
    contexts that end inside a 64-key chunk and on its last key."""
    h = qa.QorusHeader(vocab=700, dim=128 * n_heads, hidden=1024, n_layers=1, n_heads=n_heads, n_kv=n_kv,
                       max_seq=256)
    m, blob, kv = build(qa, tmp_path, h, 21 + n_heads, P)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        t = 5
        for pos in (P, P + 1):
            tok_ref, lg_ref = ref.step(t, pos)
            lg = m.forward([t], pos)
            assert rel_err(lg, lg_ref) <= 1e-4, pos
            assert int(np.argmax(lg)) == tok_ref
            t = tok_ref
    finally:
        m.close()


def test_decode_short_context_and_tails(qa, tmp_path):
    """Positions 0..9: softmax over N < 8 and N % 8 != 0 keys (the reference's
    libm tail), GQA group 2, three layers."""
    h = qa.QorusHeader(vocab=300, dim=256, hidden=512, n_layers=3, n_heads=2, n_kv=1, max_seq=64)
    m, blob, kv = build(qa, tmp_path, h, 12, 0)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        t = 3
        for pos in range(10):
            tok_ref, lg_ref = ref.step(t, pos)
            lg = m.forward([t], pos)
            assert rel_err(lg, lg_ref) <= 1e-4, pos
            assert int(np.argmax(lg)) == tok_ref
            t = tok_ref
    finally:
        m.close()


def test_forward_multi_token_matches_steps(qa, tmp_path):
    """llama_forward with seq_len > 1 equals token-by-token steps."""
    h = qa.QorusHeader(vocab=500, dim=256, hidden=512, n_layers=2, n_heads=2, n_kv=2, max_seq=64)
    m, blob, kv = build(qa, tmp_path, h, 13, 5)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        toks = [4, 9, 1, 400]
        lg = m.forward(toks, 5)
        for i, t in enumerate(toks):
            _, lg_ref = ref.step(t, 5 + i)
        assert rel_err(lg, lg_ref) <= 1e-4
        assert int(np.argmax(lg)) == int(np.argmax(lg_ref))
    finally:
        m.close()


def test_decode_config4_shapes_two_layers(qa, tmp_path):
    """BASELINE config 4 shapes (d 4096, GQA 32/8 x 128, FFN 14336, vocab
    128256, theta 500000, eps 1e-5, KV N(0,1) for positions 0..2046, token at
    2047) with 2 of the 32 layers."""
    h = qa.QorusHeader(vocab=128256, dim=4096, hidden=14336, n_layers=2, n_heads=32, n_kv=8, max_seq=2056)
    m, blob, kv = build(qa, tmp_path, h, 14, 2047, name="c4.qorus")
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        tok_ref, lg_ref = ref.step(42, 2047)
        lg = m.forward([42], 2047)
        print(f"config-4 shapes: rel logit error {rel_err(lg, lg_ref):.3e}")
        assert rel_err(lg, lg_ref) <= 1e-4
        assert int(np.argmax(lg)) == tok_ref
    finally:
        m.close()


def test_model_api_errors(qa, tmp_path):
    import ctypes as C
    lib = qa.lib()
    h = qa.QorusHeader(vocab=100, dim=256, hidden=512, n_layers=1, n_heads=2, n_kv=1, max_seq=32)
    m, blob, kv = build(qa, tmp_path, h, 15, 0)
    try:
        lg = np.empty(100, np.float32)
        t = np.array([1], np.uint32)
        f = lambda toks, n, pos: lib.llama_forward(C.byref(m.model), C.byref(m.ctx), toks, n, pos, lg.ctypes.data)
        assert f(None, 1, 0) == -10                   # NULL tokens -> INVALID_ARG
        assert f(t.ctypes.data, 0, 0) == -15          # seq_len 0 -> INVALID_SIZE
        assert f(t.ctypes.data, 33, 0) == -15         # > max_seq -> INVALID_SIZE
        assert f(t.ctypes.data, 1, 32) == -10         # pos >= max_seq -> INVALID_ARG
        bad = np.array([100], np.uint32)
        assert f(bad.ctypes.data, 1, 0) == -10        # token >= vocab -> INVALID_ARG
        out = C.c_uint32()
        assert lib.q_sample_token(lg.ctypes.data, 100, -1.0, 0, 0.0, C.byref(out), None) == -10
        lg[:] = 0
        lg[37] = 5.0
        lg[90] = 5.0
        assert lib.q_sample_token(lg.ctypes.data, 100, 0.0, 0, 0.0, C.byref(out), None) == 0
        assert out.value == 37
    finally:
        m.close()


def test_decode_unfused_wide_dim(qa, tmp_path):
    """d_model 4352 (136 blocks, above the fused kernels' 128): the layer
    runs on the generic GEMV launches (RMSNorm + digit prep, Q|K|V with RoPE
    and head-strided cache stores on the two-wave K split, residual
    epilogues), GQA 34/17."""
    h = qa.QorusHeader(vocab=300, dim=4352, hidden=1024, n_layers=2, n_heads=34, n_kv=17, max_seq=64)
    P = 20
    m, blob, kv = build(qa, tmp_path, h, 15, P, name="wide.qorus")
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        t = 5
        for pos in range(P, P + 3):
            tok_ref, lg_ref = ref.step(t, pos)
            lg = m.forward([t], pos)
            assert rel_err(lg, lg_ref) <= 1e-4, pos
            assert int(np.argmax(lg)) == tok_ref
            t = tok_ref
        kv_gpu = m.download_kv().reshape(kv.shape)
        for l in range(h.n_layers):
            assert rel_err(kv_gpu[l, :, P], ref.kv[l, :, P]) <= 1e-4
    finally:
        m.close()


def test_build_graph_rejects_unbuilt_configs(qa, tmp_path):
    """GQA groups other than 1/2/4/8 are refused at llama_build_graph with
    Q_ERR_INVALID_CONFIG (not at the first step)."""
    for i, h in enumerate([qa.QorusHeader(vocab=50, dim=384, hidden=256, n_layers=1, n_heads=3, n_kv=1, max_seq=16),
                           qa.QorusHeader(vocab=50, dim=1536, hidden=256, n_layers=1, n_heads=12, n_kv=2,
                                          max_seq=16)]):
        path = tmp_path / f"bad{i}.qorus"
        qa.synthetic.write_synthetic_model(path, h, 16)
        with pytest.raises(qa.QorusError, match="INVALID_CONFIG"):
            qa.Model(path)


def test_decode_unfused_d8448(qa, tmp_path):
    """d_model 8448 (264 blocks): Q|K|V and the LM head take fp32 x with the
    RMSNorm in the prologue of the 7-wave GEMV, whose lanes each convert the
    one block they consume (GQA 66/33)."""
    h = qa.QorusHeader(vocab=256, dim=8448, hidden=512, n_layers=1, n_heads=66, n_kv=33, max_seq=16)
    P = 5
    m, blob, kv = build(qa, tmp_path, h, 17, P, name="d8448.qorus")
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        t = 3
        for pos in range(P, P + 2):
            tok_ref, lg_ref = ref.step(t, pos)
            lg = m.forward([t], pos)
            assert rel_err(lg, lg_ref) <= 1e-4, pos
            assert int(np.argmax(lg)) == tok_ref
            t = tok_ref
    finally:
        m.close()


def test_generate_sampled_matches_host_loop(qa, tmp_path):
    """qh_llama_generate_sampled (sampling on the device, only the tokens
    leave it) equals a host loop of llama_forward + q_sample_token on the
    same thread's RNG stream with 32-byte-aligned logits, for temperature
    with top-k, top-p, both, and neither; temperature 0 is the greedy
    generation."""
    h = qa.QorusHeader(vocab=1000, dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv=1, max_seq=256)
    P, n = 50, 8
    m, blob, kv = build(qa, tmp_path, h, 21, P)
    lib = qa.lib()
    buf = orc.aligned_empty((h.vocab,), np.float32, 64)
    try:
        for T, k, p in ((0.8, 40, 0.0), (1.0, 0, 0.9), (0.7, 50, 0.95), (1.2, 0, 0.0), (0.0, 0, 0.0)):
            m.upload_kv(kv)
            lib.qh_sample_set_state(2468)
            toks, ms = m.generate_sampled(7, P, n, T, k, p)
            assert ms > 0
            m.upload_kv(kv)
            lib.qh_sample_set_state(2468)
            want, t = [], 7
            for i in range(n):
                buf[:] = m.forward([t], P + i)
                out = C.c_uint32()
                assert lib.q_sample_token(buf.ctypes.data, h.vocab, T, k, p, C.byref(out), None) == 0
                t = out.value
                want.append(t)
            assert toks.tolist() == want, (T, k, p)
    finally:
        m.close()
