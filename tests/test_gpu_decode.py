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


@pytest.mark.parametrize("P", [4100, 9100])
def test_decode_long_context(qa, tmp_path, P):
    """Contexts past the config-4 one: 4101 keys (65 score chunks: the
    chunk-max reduction takes two rounds of 64) and 9101 keys (143 score
    chunks, 36 P.V chunks: the combine sums its partials in two rounds of
    32), then greedy steps on the device against the oracle's."""
    h = qa.QorusHeader(vocab=800, dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv=1, max_seq=P + 16)
    m, blob, kv = build(qa, tmp_path, h, 17, P)
    try:
        ref = orc.DecodeOracle(blob, kv.copy())
        tok_ref, lg_ref = ref.step(5, P)
        lg = m.forward([5], P)
        assert rel_err(lg, lg_ref) <= 1e-4
        assert int(np.argmax(lg)) == tok_ref
        kv_gpu = m.download_kv().reshape(kv.shape)
        for l in range(h.n_layers):
            assert rel_err(kv_gpu[l, :, P], ref.kv[l, :, P]) <= 1e-4
        n = 4
        toks, _ = m.generate(tok_ref, P + 1, n)
        want, t = [], tok_ref
        for i in range(n):
            t, _ = ref.step(t, P + 1 + i)
            want.append(t)
        assert toks.tolist() == want
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
    """GQA groups other than 1/2/4/8, and FFN widths above 32768 (the prefill
    GEMM's row limit), are refused at llama_build_graph with
    Q_ERR_INVALID_CONFIG (not at the first step or prompt)."""
    for i, h in enumerate([qa.QorusHeader(vocab=50, dim=384, hidden=256, n_layers=1, n_heads=3, n_kv=1, max_seq=16),
                           qa.QorusHeader(vocab=50, dim=1536, hidden=256, n_layers=1, n_heads=12, n_kv=2,
                                          max_seq=16),
                           qa.QorusHeader(vocab=50, dim=128, hidden=32800, n_layers=1, n_heads=1, n_kv=1,
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


def _q4_rows(blob, lay, name, rows, cols):
    """Writable [rows, cols/32, 20] view of a Q4_0 matrix inside a model blob."""
    off = lay[name]
    return blob[off: off + rows * (cols // 32) * 20].reshape(rows, cols // 32, 20)


def _scales(mat):
    return mat[:, :, 16:].view(np.float32)[:, :, 0]


def _zero_cols(mat, cols):
    for j in cols:
        b, e = divmod(int(j), 32)
        if e & 1:
            mat[:, b, e >> 1] = (mat[:, b, e >> 1] & 0x0F) | 0x80
        else:
            mat[:, b, e >> 1] = (mat[:, b, e >> 1] & 0xF0) | 0x08


def test_decode_outliers_at_wo_and_w_down_inputs(qa, tmp_path):
    """Activation outliers that meet zero weights at the two GEMV inputs the
    decode step converts itself: the attention output (digits made by the
    attention combine, the Wo input) and the SwiGLU product (converted in
    the W_down launch).  Config-4 widths (d 4096, GQA 32/8, FFN 14336),
    2 layers, vocabulary cut to 512.
      * Layer 0: Wo's scales are 0, so x1 is the token's embedding row and
        the FFN input is known on the host.  In five 32-row blocks of the
        FFN, 2, 3, 4 and 6 rows (and 4 rows of mixed sizes) get W_gate
        scales of the sign that makes gate_i > 0 and W_up scales 1e3 times
        (1e4..1e1 for the mixed block) larger: h_i = silu(g_i) u_i are
        outliers, and W_down has zero weights (nibble 8) in those columns.
      * Layer 1: the cached V rows hold +-1e4 in 2, 3, 4 and 6 dimensions of
        the four 32-dimension blocks of each head (in every head), so the
        attention output carries them in every block of the Wo input, and
        Wo has zero weights there.
    With the outliers' blocks on the GEMV's second digit level, logits and
    the written cache rows stay within 1e-5 of the oracle (the AVX2-order
    CPU step); on the first level alone the other elements of those blocks
    lose their low bits (errors of 1e-4 and more)."""
    h = qa.QorusHeader(vocab=512, dim=4096, hidden=14336, n_layers=2, n_heads=32, n_kv=8, max_seq=320)
    P, tok = 300, 17
    path = tmp_path / "adv.qorus"
    qa.synthetic.write_synthetic_model(path, h, 31)
    blob = np.fromfile(path, dtype=np.uint8)
    lay = qa.model_file.model_layout(h)
    d, hid = h.dim, h.hidden
    # layer 0: Wo contributes exactly 0
    _scales(_q4_rows(blob, lay, "0.wo", d, d))[:] = 0.0
    emb = blob[lay["token_embd"]: lay["token_embd"] + h.vocab * d * 4].view(np.float32).reshape(h.vocab, d)
    nw = blob[lay["0.ffn_norm"]: lay["0.ffn_norm"] + d * 4].view(np.float32)
    x = emb[tok].astype(np.float64)
    xn = x / np.sqrt(np.mean(x * x) + h.eps) * nw
    wg = _q4_rows(blob, lay, "0.w_gate", hid, d)
    wu = _q4_rows(blob, lay, "0.w_up", hid, d)
    g = orc.dequant_np(wg.reshape(hid, -1)) @ xn
    rng = orc.rng_for(31, 7)
    blocks = rng.choice(hid // 32, 5, replace=False)
    outl = []
    for b, (n, f) in zip(blocks, [(2, [1e3] * 2), (3, [1e3] * 3), (4, [1e3] * 4), (6, [1e3] * 6),
                                  (4, [1e4, 1e3, 1e2, 1e1])]):
        rows = [32 * int(b) + e for e in rng.permutation(32) if abs(g[32 * int(b) + e]) > 0.5 * g.std()][:n]
        assert len(rows) == n
        for i, fi in zip(rows, f):
            if g[i] < 0:
                _scales(wg)[i] *= -1.0
            _scales(wu)[i] *= np.float32(fi)
            outl.append(i)
    _zero_cols(_q4_rows(blob, lay, "0.w_down", d, hid), outl)
    # layer 1: V outliers in every block of every head, zero Wo columns
    hd = h.head_dim
    dims = [e for blk, n in enumerate((2, 3, 4, 6)) for e in (32 * blk + rng.permutation(32)[:n])]
    _zero_cols(_q4_rows(blob, lay, "1.wo", d, d), [hh * hd + e for hh in range(h.n_heads) for e in dims])
    blob.tofile(path)
    kv = np.zeros((h.n_layers, h.n_kv, h.max_seq, 2, hd), np.float32)
    kv[:, :, :P] = orc.rng_for(31, 99).standard_normal((h.n_layers, h.n_kv, P, 2, hd), dtype=np.float32)
    for i, e in enumerate(dims):
        kv[1, :, :P, 1, e] = 1e4 if i % 2 == 0 else -1e4
    m = qa.Model(path)
    try:
        m.upload_kv(kv)
        ref = orc.DecodeOracle(blob, kv.copy())
        tok_ref, lg_ref = ref.step(tok, P)
        lg = m.forward([tok], P)
        kv_gpu = m.download_kv().reshape(kv.shape)
        e_lg = rel_err(lg, lg_ref)
        e_kv = [rel_err(kv_gpu[l, :, P], ref.kv[l, :, P]) for l in range(h.n_layers)]
        print(f"outliers at the Wo / W_down inputs: logits {e_lg:.3e}, cache rows {e_kv}")
        assert int(np.argmax(lg)) == tok_ref
        assert e_lg <= 1e-5
        assert max(e_kv) <= 1e-5
    finally:
        m.close()


def _scratch_dir(tmp_path, need):
    """/dev/shm when it holds the file (the bench's choice), else tmp_path."""
    import shutil
    import tempfile
    try:
        if shutil.disk_usage("/dev/shm").free > need * 1.2:
            return tempfile.mkdtemp(prefix="qorus_test_", dir="/dev/shm")
    except OSError:
        pass
    return str(tmp_path)


def test_decode_config4_full_depth(qa, tmp_path):
    """BASELINE config 4 at its own depth: the 32-layer Llama-3-8B-shaped
    model (vocab 128256, Q4_0 LM head), KV N(0,1) at positions 0..2046, the
    token at 2047.  The first step's logits (1e-4 of the largest) and the
    cache rows it writes in all 32 layers (1e-4 of each row's largest)
    against the oracle, then three greedy tokens in all (one llama_forward,
    two steps of the device generation loop) equal to the oracle's."""
    import os
    import shutil
    h = qa.QorusHeader(vocab=128256, dim=4096, hidden=14336, n_layers=32, n_heads=32, n_kv=8, max_seq=2056)
    P = 2047
    d = _scratch_dir(tmp_path, qa.model_layout(h)["_size"])
    path = os.path.join(d, "c4_full.qorus")
    m = None
    orc.set_threads(min(16, os.cpu_count() or 1))
    try:
        qa.synthetic.write_synthetic_model(path, h, 2024)
        m = qa.Model(path)
        kv = np.zeros((h.n_layers, h.n_kv, h.max_seq, 2, 128), np.float32)
        kv[:, :, :P] = orc.rng_for(2025).standard_normal((h.n_layers, h.n_kv, P, 2, 128), dtype=np.float32)
        m.upload_kv(kv)
        ref = orc.DecodeOracle(np.memmap(path, dtype=np.uint8, mode="r"), kv)
        t0 = 1
        lg = m.forward([t0], P)
        tok1, lg_ref = ref.step(t0, P)
        e = rel_err(lg, lg_ref)
        kv_gpu = m.download_kv().reshape(kv.shape)
        ek = max(rel_err(kv_gpu[l, :, P], ref.kv[l, :, P]) for l in range(h.n_layers))
        print(f"config 4, 32 layers: logits {e:.3e}, cache rows {ek:.3e}")
        assert int(np.argmax(lg)) == tok1
        assert e <= 1e-4 and ek <= 1e-4
        toks, _ = m.generate(tok1, P + 1, 2)
        tok2, _ = ref.step(tok1, P + 1)
        tok3, _ = ref.step(tok2, P + 2)
        assert toks.tolist() == [tok2, tok3]
    finally:
        orc.set_threads(1)
        if m is not None:
            m.close()
        if d != str(tmp_path):
            shutil.rmtree(d, ignore_errors=True)


def _hip_free_bytes():
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_no_device_allocation_after_build_graph(qa, tmp_path):
    """After llama_build_graph (and the first decode step, which captures the
    step's graph), the first prompt through llama_forward, the first device
    sampled generation and a GEMV wider than the in-kernel conversion with a
    NULL workspace allocate no device memory: hipMemGetInfo's free bytes do
    not change across them."""
    import ctypes as C
    h = qa.QorusHeader(vocab=1000, dim=512, hidden=1024, n_layers=2, n_heads=4, n_kv=1, max_seq=256)
    m, blob, kv = build(qa, tmp_path, h, 41, 20)
    lib = qa.lib()
    M, N = 64, 32768
    rng = orc.rng_for(41, 5)
    dW = qa.DeviceBuffer.from_numpy(orc.gen_q4(M, N, rng))
    dx = qa.DeviceBuffer.from_numpy(orc.gen_f32(N, rng))
    dy = qa.DeviceBuffer(M * 4)
    t = qa.q4_tensor(dW.ptr, M, N)
    try:
        m.forward([3], 20)  # the decode step's graph is captured here
        qa.check(lib.qh_device_synchronize())
        f0 = _hip_free_bytes()
        m.forward([int(v) for v in rng.integers(0, h.vocab, 40)], 21)      # first prompt
        f1 = _hip_free_bytes()
        m.generate_sampled(7, 61, 4, 0.8, 40, 0.95)                        # first sampled loop
        f2 = _hip_free_bytes()
        qa.check(lib.qh_gemv_q4_f32(t.addr, dx.ptr, dy.ptr, None, None), "gemv, NULL workspace")
        qa.check(lib.qh_device_synchronize())
        f3 = _hip_free_bytes()
        print(f"free bytes: {f0} {f1} {f2} {f3}")
        assert f0 == f1 == f2 == f3, (f0 - f1, f1 - f2, f2 - f3)
        # the wide GEMV ran on the library's workspace: its result is right
        y64, cond = orc.gemv_f64(orc.gen_q4(M, N, orc.rng_for(41, 5)), M, N, dx.download(np.float32, (N,)))
        assert np.max(np.abs(dy.download(np.float32, (M,)) - y64) / cond) <= 1e-5
    finally:
        m.close()
