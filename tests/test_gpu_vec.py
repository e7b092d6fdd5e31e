"""GPU parity of the vector ops that feed the GEMV in the decode step,
through the C-ABI (host-pointer qorus.h entry points and device qh_* ones).

Bars, written out:
  RoPE, add, mul, SiLU on its first N&~7 elements: bit-exact with the oracle
    (the same IEEE operations in the same order);
  SiLU/softmax N%8 tails (libm expf there, device expf here): <= 2 ulp;
  RMSNorm: relative error <= 2e-6 (reduction order + reciprocal-sqrt seed);
  softmax (q_softmax_f32_avx2, qh_softmax_f32[_ws]): bit-exact for N % 8 == 0
    (the reference's eight lane sums and tree); with a tail, the tail's expf
    may differ by an ulp and move the sum, so <= 2 ulp everywhere;
  fused softmax + argmax (qh_softmax_argmax_f32_ws, the LM-head form, a
    tree sum over the chip): relative error <= 2e-6, the same zero pattern;
  argmax: identical index, first index on ties.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def host(n):
    return orc.aligned_empty((n,), np.float32)


@pytest.mark.parametrize("N", [8, 128, 4096, 14336])
def test_rmsnorm(qa, N):
    rng = orc.rng_for(201, N)
    x, w = orc.aligned_copy(orc.gen_f32(N, rng)), orc.aligned_copy(orc.gen_f32(N, rng))
    y = host(N)
    assert qa.lib().q_rmsnorm_f32_avx2(x.ctypes.data, w.ctypes.data, y.ctypes.data, N, 1e-5) == 0
    want = orc.rmsnorm(x, w, 1e-5)
    assert np.max(np.abs(y - want) / (np.abs(want) + 1e-30)) <= 2e-6
    # device entry point gives the same bits as the host one
    dx, dw, dy = (qa.DeviceBuffer.from_numpy(a) for a in (x, w, y))
    qa.check(qa.lib().qh_rmsnorm_f32(dx.ptr, dw.ptr, dy.ptr, N, 1e-5, None))
    qa.check(qa.lib().qh_device_synchronize())
    assert np.array_equal(bits(dy.download(np.float32, (N,))), bits(y))


def test_rope_bitexact(qa):
    rng = orc.rng_for(202)
    for pos in (0, 1, 2047, 8191):
        c, s = (orc.aligned_copy(t) for t in orc.rope_tables(500000.0, 128, pos))
        x = orc.aligned_copy(orc.gen_f32(128, rng))
        y = host(128)
        assert qa.lib().q_rope_f32_avx2(x.ctypes.data, c.ctypes.data, s.ctypes.data, y.ctypes.data, 128) == 0
        assert np.array_equal(bits(y), bits(orc.rope(x, c, s)))
    # batched device form: 40 heads (32 q + 8 k) with one table pair
    c, s = orc.rope_tables(500000.0, 128, 2047)
    X = orc.gen_f32(40 * 128, rng)
    dX, dc, ds, dY = (qa.DeviceBuffer.from_numpy(a) for a in (X, c, s, np.zeros_like(X)))
    qa.check(qa.lib().qh_rope_f32(dX.ptr, dc.ptr, ds.ptr, dY.ptr, 128, 40, None))
    qa.check(qa.lib().qh_device_synchronize())
    Y = dY.download(np.float32, (40 * 128,))
    want = np.concatenate([orc.rope(X[h * 128:(h + 1) * 128], c, s) for h in range(40)])
    assert np.array_equal(bits(Y), bits(want))


@pytest.mark.parametrize("N", [1, 5, 8, 29, 4096, 14336])
def test_silu(qa, N):
    rng = orc.rng_for(203, N)
    x = orc.aligned_copy((rng.random(N, dtype=np.float32) * 24 - 12).astype(np.float32))
    y = host(N)
    assert qa.lib().q_silu_f32_avx2(x.ctypes.data, y.ctypes.data, N) == 0
    want = orc.silu(x)
    nv = N & ~7 if N >= 8 else 0
    assert np.array_equal(bits(y[:nv]), bits(want[:nv]))
    assert np.all(ulp_diff(y[nv:], want[nv:]) <= 2)


def test_silu_mul_fused(qa):
    rng = orc.rng_for(204)
    N = 14336
    g, u = orc.gen_f32(N, rng) * 3, orc.gen_f32(N, rng)
    dg, du, do = qa.DeviceBuffer.from_numpy(g), qa.DeviceBuffer.from_numpy(u), qa.DeviceBuffer(N * 4)
    qa.check(qa.lib().qh_silu_mul_f32(dg.ptr, du.ptr, do.ptr, N, None))
    qa.check(qa.lib().qh_device_synchronize())
    assert np.array_equal(bits(do.download(np.float32, (N,))), bits(orc.mul(orc.silu(g), u)))


def check_softmax(y, want, N):
    """Bit-exact when N % 8 == 0, else within 2 ulp (the libm tail)."""
    if N >= 8 and N % 8 == 0:
        assert np.array_equal(bits(y), bits(want))
    else:
        assert np.array_equal(y == 0, want == 0)
        assert np.all(ulp_diff(y, want) <= 2)


SOFTMAX_N = [1, 5, 8, 71, 2048, 4096, 16384, 128256, 131077]


@pytest.mark.parametrize("N", SOFTMAX_N)
def test_softmax(qa, N):
    """q_softmax_f32_avx2 in the reference's order: N(0, 2^2) logits (a few
    nonzero exponentials: the sparse lane sums) and near-flat ones (every
    exponential nonzero: the dense lane sums), against the oracle and, where
    built, the reference's own q_softmax_f32_avx2."""
    rng = orc.rng_for(205, N)
    for scale in (2.0, 0.01):
        x = orc.aligned_copy((orc.gen_f32(N, rng) * scale).astype(np.float32))
        y = host(N)
        assert qa.lib().q_softmax_f32_avx2(x.ctypes.data, y.ctypes.data, N) == 0
        want = orc.softmax(x)
        check_softmax(y, want, N)
        if orc.ref_available():
            rc, ref = orc.ref_softmax(x)
            assert rc == 0
            check_softmax(y, ref, N)
        assert abs(float(y.sum(dtype=np.float64)) - 1.0) < 1e-4


def test_add_mul_bitexact(qa):
    rng = orc.rng_for(206)
    N = 4096
    a, b = orc.aligned_copy(orc.gen_f32(N, rng)), orc.aligned_copy(orc.gen_f32(N, rng))
    o = host(N)
    ta, tb, to = qa.f32_tensor(a.ctypes.data, N), qa.f32_tensor(b.ctypes.data, N), qa.f32_tensor(o.ctypes.data, N)
    assert qa.lib().q_add_f32_avx2(ta.addr, tb.addr, to.addr) == 0
    assert np.array_equal(bits(o), bits(orc.add(a, b)))
    assert qa.lib().q_mul_f32_avx2(ta.addr, tb.addr, to.addr) == 0
    assert np.array_equal(bits(o), bits(orc.mul(a, b)))
    # in place (output aliases a), as the reference allows
    a0 = a.copy()
    assert qa.lib().q_add_f32_avx2(ta.addr, tb.addr, ta.addr) == 0
    assert np.array_equal(bits(a), bits(orc.add(a0, b)))


def test_argmax(qa):
    rng = orc.rng_for(207)
    cases = [orc.gen_f32(128256, rng), np.array([1, 5, 5, 2, 5], np.float32),
             np.array([np.nan, 3, 4], np.float32), np.array([2, np.nan, 7, 7], np.float32),
             np.full(1000, -np.inf, np.float32), np.array([3.0], np.float32)]
    out = qa.DeviceBuffer(4)
    for x in cases:
        dx = qa.DeviceBuffer.from_numpy(x)
        qa.check(qa.lib().qh_argmax_f32(dx.ptr, x.size, out.ptr, None))
        qa.check(qa.lib().qh_device_synchronize())
        assert int(out.download(np.uint32, (1,))[0]) == orc.argmax(x)


def test_argmax_multi_workgroup_cases(qa):
    """N >= 16384 takes the multi-workgroup path (per-slice partials, then a
    combine): ties across slices keep the first index, NaN never wins, NaN
    at index 0 gives 0, all -inf gives 0; _ws form with its own workspace."""
    lib = qa.lib()
    N = 128256
    rng = orc.rng_for(209)
    base = orc.gen_f32(N, rng)
    tie = base.copy()
    tie[[5000, 70000, 127000]] = 50.0                 # tie across three slices
    nan_mid = base.copy()
    nan_mid[[3, 64000]] = np.nan
    nan_mid[90000] = 60.0
    nan0 = base.copy()
    nan0[0] = np.nan
    cases = [base, tie, nan_mid, nan0, np.full(N, -np.inf, np.float32), np.zeros(N, np.float32),
             np.concatenate([np.full(N - 1, -1.0, np.float32), [np.float32(-0.5)]])]
    out = qa.DeviceBuffer(4)
    ws = qa.DeviceBuffer(lib.qh_argmax_workspace_bytes(N))
    for x in cases:
        dx = qa.DeviceBuffer.from_numpy(x)
        for use_ws in (False, True):
            if use_ws:
                qa.check(lib.qh_argmax_f32_ws(dx.ptr, N, out.ptr, ws.ptr, None))
            else:
                qa.check(lib.qh_argmax_f32(dx.ptr, N, out.ptr, None))
            qa.check(lib.qh_device_synchronize())
            assert int(out.download(np.uint32, (1,))[0]) == orc.argmax(x)


@pytest.mark.parametrize("N", [16384, 128256, 131077, 3000000])
def test_softmax_device_entry_points(qa, N):
    """qh_softmax_f32 (library workspace) and qh_softmax_f32_ws (caller's,
    in place and out of place) in the reference's order: the oracle's bits
    (N % 8 == 0) or within 2 ulp (N % 8 tails), on sparse and near-flat
    logits; 3,000,000 runs the dense lane sums without a list."""
    lib = qa.lib()
    rng = orc.rng_for(211, N)
    for scale in (3.0, 0.01):
        x = (orc.gen_f32(N, rng) * scale).astype(np.float32)
        want = orc.softmax(orc.aligned_copy(x))
        dx = qa.DeviceBuffer.from_numpy(x)
        dy = qa.DeviceBuffer(N * 4)
        ws = qa.DeviceBuffer(lib.qh_softmax_workspace_bytes(N))
        for mode in ("plain", "ws", "inplace"):
            if mode == "plain":
                qa.check(lib.qh_softmax_f32(dx.ptr, dy.ptr, N, None))
            elif mode == "ws":
                qa.check(lib.qh_softmax_f32_ws(dx.ptr, dy.ptr, N, ws.ptr, None))
            else:
                dz = qa.DeviceBuffer.from_numpy(x)
                qa.check(lib.qh_softmax_f32_ws(dz.ptr, dz.ptr, N, ws.ptr, None))
                dy = dz
            qa.check(lib.qh_device_synchronize())
            check_softmax(dy.download(np.float32, (N,)), want, N)


def test_softmax_argmax_fused(qa):
    """qh_softmax_argmax_f32_ws: the probabilities within 2e-6 of the
    oracle's (a tree sum over the chip) with the same zero pattern, and the
    index the reference argmax of x (first index of the maximum, NaN never
    wins, NaN at index 0 gives 0) on the multi-workgroup path and on the
    small-N path; aliasing is refused."""
    lib = qa.lib()
    rng = orc.rng_for(213)
    cases = []
    for N in (100, 16384, 128256, 131077):
        base = (orc.gen_f32(N, rng) * 3).astype(np.float32)
        cases.append(base)
        if N >= 16384:
            tie = base.copy()
            tie[[N // 7, N // 2, N - 3]] = 50.0
            nan_mid = base.copy()
            nan_mid[[3, N // 2]] = np.nan
            nan_mid[N - 100] = 60.0
            nan0 = base.copy()
            nan0[0] = np.nan
            cases += [tie, nan_mid, nan0, np.zeros(N, np.float32)]
    for x in cases:
        N = x.size
        dx = qa.DeviceBuffer.from_numpy(x)
        dy, dy2 = qa.DeviceBuffer(N * 4), qa.DeviceBuffer(N * 4)
        ws = qa.DeviceBuffer(lib.qh_softmax_workspace_bytes(N))
        out = qa.DeviceBuffer(4)
        qa.check(lib.qh_softmax_argmax_f32_ws(dx.ptr, dy.ptr, N, out.ptr, ws.ptr, None))
        qa.check(lib.qh_device_synchronize())
        y = dy.download(np.float32, (N,))
        if np.isfinite(x).all():
            want = orc.softmax(orc.aligned_copy(x))
            assert np.array_equal(y == 0, want == 0)
            nz = want != 0
            assert np.max(np.abs(y[nz] - want[nz]) / want[nz]) <= 2e-6
        assert int(out.download(np.uint32, (1,))[0]) == orc.argmax(x)
    from qorus_amd import _lib as L
    assert lib.qh_softmax_argmax_f32_ws(dx.ptr, dx.ptr, N, out.ptr, ws.ptr, None) == L.Q_ERR_ALIASING


@pytest.mark.parametrize("M,N", [(20000, 4096), (16384, 2080), (5000, 4096), (17000, 1024)])
def test_gemv_softmax_argmax(qa, M, N):
    """qh_gemv_q4_f32_softmax_argmax: logits and probabilities bit-identical
    to qh_gemv_q4_f32_multi followed by qh_softmax_argmax_f32_ws, and the
    index the reference argmax of the logits, including a three-way tie for
    the maximum (identical weight rows give identical logits: the first row
    wins).  The first two shapes take the GEMV's argmax partials, the others
    the separate passes."""
    from qorus_amd import _lib as L
    from qorus_amd import synthetic as syn
    lib = qa.lib()
    rng = orc.rng_for(227, M, N)
    w = syn.gen_q4(M, N, rng)
    x = syn.gen_f32(N, rng)
    dw = qa.DeviceBuffer.from_numpy(w)
    dx = qa.DeviceBuffer.from_numpy(x)
    W = qa.q4_tensor(dw.ptr, M, N)
    lg, pr = qa.DeviceBuffer(M * 4), qa.DeviceBuffer(M * 4)
    lg2, pr2 = qa.DeviceBuffer(M * 4), qa.DeviceBuffer(M * 4)
    idx, idx2 = qa.DeviceBuffer(4), qa.DeviceBuffer(4)
    ws = qa.DeviceBuffer(lib.qh_gemv_softmax_workspace_bytes(M))
    ws2 = qa.DeviceBuffer(lib.qh_softmax_workspace_bytes(M))
    for tie in (False, True):
        if tie:
            # rows 100 and M - 7 become copies of the current maximum's row
            r = orc.argmax(lg.download(np.float32, (M,)))
            w[[100, M - 7]] = w[r]
            dw = qa.DeviceBuffer.from_numpy(w)
            W = qa.q4_tensor(dw.ptr, M, N)
        qa.check(lib.qh_gemv_q4_f32_softmax_argmax(W.addr, dx.ptr, lg.ptr, pr.ptr, idx.ptr, ws.ptr, None))
        ys = (C.c_void_p * 1)(lg2.ptr)
        Ws = (C.c_void_p * 1)(W.addr)
        qa.check(lib.qh_gemv_q4_f32_multi(Ws, None, ys, 1, dx.ptr, None, None))
        qa.check(lib.qh_softmax_argmax_f32_ws(lg2.ptr, pr2.ptr, M, idx2.ptr, ws2.ptr, None))
        qa.check(lib.qh_device_synchronize())
        logits = lg.download(np.float32, (M,))
        assert np.array_equal(bits(logits), bits(lg2.download(np.float32, (M,))))
        assert np.array_equal(bits(pr.download(np.float32, (M,))), bits(pr2.download(np.float32, (M,))))
        got = int(idx.download(np.uint32, (1,))[0])
        assert got == int(idx2.download(np.uint32, (1,))[0]) == orc.argmax(logits)
        if tie:
            assert got == min(100, r)
    # a NaN input makes every logit NaN: index 0 (nothing compares greater)
    dn = qa.DeviceBuffer.from_numpy(np.full(N, np.nan, np.float32))
    qa.check(lib.qh_gemv_q4_f32_softmax_argmax(W.addr, dn.ptr, lg.ptr, pr.ptr, idx.ptr, ws.ptr, None))
    qa.check(lib.qh_device_synchronize())
    assert np.all(np.isnan(lg.download(np.float32, (M,))))
    assert int(idx.download(np.uint32, (1,))[0]) == 0
    assert lib.qh_gemv_q4_f32_softmax_argmax(W.addr, dx.ptr, lg.ptr, lg.ptr, idx.ptr, ws.ptr, None) == \
        L.Q_ERR_ALIASING
    assert lib.qh_gemv_q4_f32_softmax_argmax(W.addr, dx.ptr, lg.ptr, pr.ptr, idx.ptr, None, None) == \
        L.Q_ERR_INVALID_ARG


# ------------------------------------------------------------ fp32 matmul --

def _mat_tensor(qa, arr, ne0, ne1, nb0, nb1=4):
    from qorus_amd._lib import _AlignedTensor
    return _AlignedTensor(arr.ctypes.data, (ne0, ne1, 1, 1), (nb0, nb1, 4, 4), qa.Q_F32)


@pytest.mark.parametrize("M,K,N", [(1, 128, 2048), (32, 128, 33), (5, 31, 7), (3, 33, 4), (7, 200, 9),
                                   (64, 1024, 64), (1, 1, 1)])
def test_matmul_f32_bitexact(qa, M, K, N):
    """q_matmul_f32_avx2 (reference matmul_fp32.c): dense, transposed-B and
    strided variants, bit-exact with the oracle's restatement (itself
    bit-identical to the reference build, see test_oracle)."""
    import ctypes as C
    from qorus_amd.model import QContext
    lib = qa.lib()
    rng = orc.rng_for(M * 1000 + K, N)
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = rng.standard_normal((K, N), dtype=np.float32)
    want = orc.matmul_f32(A, B)
    ctx = QContext()
    assert lib.q_alloc_arena(C.byref(ctx), K * N * 4 + 4096) == 0
    try:
        # dense
        Aa, Ba = orc.aligned_copy(A), orc.aligned_copy(B)
        Cc = orc.aligned_empty((M, N), np.float32)
        ta, tb, tc = _mat_tensor(qa, Aa, M, K, K * 4), _mat_tensor(qa, Ba, K, N, N * 4), _mat_tensor(qa, Cc, M, N, N * 4)
        assert lib.q_matmul_f32_avx2(ta.addr, tb.addr, tc.addr, C.byref(ctx)) == 0
        assert np.array_equal(bits(Cc), bits(want))
        # transposed B view: element (k, j) at Bt[j*K + k]; no arena use
        Bt = orc.aligned_copy(np.ascontiguousarray(B.T))
        head = ctx.scratch_head
        tbt = _mat_tensor(qa, Bt, K, N, 4, K * 4)
        Ct = orc.aligned_empty((M, N), np.float32)
        tct = _mat_tensor(qa, Ct, M, N, N * 4)
        assert lib.q_matmul_f32_avx2(ta.addr, tbt.addr, tct.addr, C.byref(ctx)) == 0
        if K > 1:
            assert ctx.scratch_head == head
            assert np.array_equal(bits(Ct), bits(want))
        # strided A (row stride K+5 floats) and C (row stride N+3): gaps untouched
        As = orc.aligned_empty((M, K + 5), np.float32)
        As[:, :K] = A
        As[:, K:] = np.nan
        Cs = orc.aligned_copy(np.full((M, N + 3), 7.0, np.float32))
        tas = _mat_tensor(qa, As, M, K, (K + 5) * 4)
        tcs = _mat_tensor(qa, Cs, M, N, (N + 3) * 4)
        lib.q_arena_reset(C.byref(ctx))
        assert lib.q_matmul_f32_avx2(tas.addr, tb.addr, tcs.addr, C.byref(ctx)) == 0
        assert np.array_equal(bits(Cs[:, :N]), bits(want))
        assert np.all(Cs[:, N:] == 7.0)
    finally:
        lib.q_free_memory(C.byref(ctx))


def test_matmul_f32_arena_oom(qa):
    import ctypes as C
    from qorus_amd.model import QContext
    lib = qa.lib()
    M, K, N = 4, 64, 64
    A = orc.aligned_copy(np.ones((M, K), np.float32))
    B = orc.aligned_copy(np.ones((K, N), np.float32))
    Cc = orc.aligned_empty((M, N), np.float32)
    ctx = QContext()
    assert lib.q_alloc_arena(C.byref(ctx), 1024) == 0
    try:
        ta, tb, tc = _mat_tensor(qa, A, M, K, K * 4), _mat_tensor(qa, B, K, N, N * 4), _mat_tensor(qa, Cc, M, N, N * 4)
        assert lib.q_matmul_f32_avx2(ta.addr, tb.addr, tc.addr, C.byref(ctx)) == -8  # ARENA_OOM
    finally:
        lib.q_free_memory(C.byref(ctx))


def test_gemv_softmax_argmax_errors(qa):
    """qh_gemv_q4_f32_softmax_argmax: a NULL workspace is refused with the
    other NULL arguments (before the alignment and aliasing checks), and
    operands that are not device memory of the required extent (a host x,
    host weights, a short probs buffer, a short workspace) are refused with
    Q_ERR_INVALID_ARG instead of reaching a kernel."""
    from qorus_amd import _lib as L
    lib = qa.lib()
    f = lib.qh_gemv_q4_f32_softmax_argmax
    M, N = 300, 512
    rng = orc.rng_for(233)
    dW = qa.DeviceBuffer.from_numpy(orc.gen_q4(M, N, rng))
    t = qa.q4_tensor(dW.ptr, M, N)
    dx = qa.DeviceBuffer.from_numpy(orc.gen_f32(N, rng))
    lg, pr, idx = qa.DeviceBuffer(M * 4), qa.DeviceBuffer(M * 4), qa.DeviceBuffer(4)
    ws = qa.DeviceBuffer(lib.qh_gemv_softmax_workspace_bytes(M))
    assert f(t.addr, dx.ptr, lg.ptr, pr.ptr + 4, idx.ptr, None, None) == L.Q_ERR_INVALID_ARG  # NULL workspace first
    assert f(t.addr, dx.ptr, lg.ptr, pr.ptr + 4, idx.ptr, ws.ptr, None) == L.Q_ERR_MISALIGNED
    hx = orc.aligned_copy(orc.gen_f32(N, rng))
    assert f(t.addr, hx.ctypes.data, lg.ptr, pr.ptr, idx.ptr, ws.ptr, None) == L.Q_ERR_INVALID_ARG
    hw = orc.aligned_copy(orc.gen_q4(M, N, rng).reshape(-1))
    th = qa.q4_tensor(hw.ctypes.data, M, N)
    assert f(th.addr, dx.ptr, lg.ptr, pr.ptr, idx.ptr, ws.ptr, None) == L.Q_ERR_INVALID_ARG
    short = qa.DeviceBuffer((M - 8) * 4)
    assert f(t.addr, dx.ptr, lg.ptr, short.ptr, idx.ptr, ws.ptr, None) == L.Q_ERR_INVALID_ARG
    wshort = qa.DeviceBuffer(64)
    assert f(t.addr, dx.ptr, lg.ptr, pr.ptr, idx.ptr, wshort.ptr, None) == L.Q_ERR_INVALID_ARG
    assert f(t.addr, dx.ptr, lg.ptr, pr.ptr, idx.ptr, ws.ptr, None) == 0
    assert lib.qh_device_synchronize() == 0
