"""GPU parity of the batched prefill GEMM (qh_gemm_q4_f32 / _multi) through
the C-ABI.

The reference's prefill runs q_gemv_q4_f32_avx2 once per token row
(src/models/model.c:1120-1561), so the oracle is the per-row AVX2-order
restatement (or_gemm_q4_rows) and the fp64 dot product per row.

Tolerance, written out: for every token t and output row m,
    |Y[t,m] - Y64[t,m]| / sum_k |W[m,k] X[t,k]|  <=  1e-5,
and, per token at the BASELINE widths (N >= 4096: config 5's 4096 and
14336, the GEMV tests' rule for the BASELINE shapes), the maximum of that
statistic must not exceed the AVX2 order's own maximum by more than 10%
(the MFMA accumulation order differs from the reference's eight-lane
order; both sit at the fp32 rounding level, ~1e-8, three orders of
magnitude under the bar).  Below N = 4096 the bound is three times the
AVX2 order's maximum: with few blocks the error is the rounding inside each
block's MFMA partial sum and of the scaled sum over blocks, which for
N = 96 an exact CPU emulation of that structure (exact X, one rounding per
block partial) already puts at 1.0-1.5x the AVX2 order's, and the matrix
core's own summation order adds to it (measured up to 2.2x at N = 96).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


class Gemm:
    def __init__(self, qa, Ws, Ms, N, T):
        self.qa, self.Ms, self.N, self.T = qa, Ms, N, T
        lib = qa.lib()
        self.dW = [qa.DeviceBuffer.from_numpy(np.ascontiguousarray(W)) for W in Ws]
        self.t = [qa.q4_tensor(d.ptr, M, N) for d, M in zip(self.dW, Ms)]
        self.dX = qa.DeviceBuffer(T * N * 4)
        self.dY = [qa.DeviceBuffer(T * M * 4) for M in Ms]
        self.ws = qa.DeviceBuffer(lib.qh_gemm_workspace_bytes(N, T, sum(Ms)))

    def __call__(self, X):
        qa, lib = self.qa, self.qa.lib()
        self.dX.upload(np.ascontiguousarray(X, np.float32))
        if len(self.Ms) == 1:
            qa.check(lib.qh_gemm_q4_f32(self.t[0].addr, self.dX.ptr, self.T, self.dY[0].ptr, self.ws.ptr, None))
        else:
            n = len(self.Ms)
            Ws = (C.c_void_p * n)(*[t.addr for t in self.t])
            Ys = (C.c_void_p * n)(*[d.ptr for d in self.dY])
            qa.check(lib.qh_gemm_q4_f32_multi(Ws, Ys, n, self.dX.ptr, self.T, self.ws.ptr, None))
        qa.check(lib.qh_device_synchronize())
        return [d.download(np.float32, (self.T, M)) for d, M in zip(self.dY, self.Ms)]


def check_rows(W, M, N, X, Y, tokens, slack=None):
    """fp64 + AVX2-order comparison for the given token rows."""
    if slack is None:
        slack = 1.10 if N >= 4096 else 3.0
    worst, worst_avx = 0.0, 0.0
    for t in tokens:
        y64, cond = orc.gemv_f64(W, M, N, X[t])
        cond = np.maximum(cond, 1e-300)
        e = float(np.max(np.abs(Y[t].astype(np.float64) - y64) / cond))
        ea = float(np.max(np.abs(orc.gemv(W, M, N, X[t]).astype(np.float64) - y64) / cond))
        assert e <= 1e-5, (t, e)
        assert e <= ea * slack, (t, e, ea)
        worst, worst_avx = max(worst, e), max(worst_avx, ea)
    return worst, worst_avx


@pytest.mark.parametrize("M,N,T", [
    (256, 4096, 128),    # one tile
    (300, 4096, 77),     # ragged rows and tokens
    (64, 96, 5),         # odd block count (3), tiny
    (1000, 2080, 130),   # odd block count (65), two token tiles
    (512, 14336, 40),    # down-projection width, split-K
    (40, 8192, 257),     # few rows, three token tiles (no XCD order)
    (300, 4096, 16),     # 16-token tiles, K split
    (1024, 4096, 20),    # 32-token tiles
    (512, 14336, 64),    # 64-token tiles, a deep K split
    (2048, 14336, 9),    # 16-token tiles, K split 16
])
def test_gemm_vs_oracle(qa, M, N, T):
    rng = orc.rng_for(M * 7 + N, T)
    W = orc.gen_q4(M, N, rng)
    X = rng.standard_normal((T, N), dtype=np.float32)
    (Y,) = Gemm(qa, [W], [M], N, T)(X)
    assert Y.shape == (T, M) and np.all(np.isfinite(Y))
    toks = sorted(set([0, T - 1] + list(range(0, T, max(1, T // 8)))))
    e, ea = check_rows(W, M, N, X, Y, toks)
    print(f"M={M} N={N} T={T}: max err/cond {e:.3e} (avx2 order {ea:.3e})")
    # whole matrix against the per-row AVX2-order oracle
    Yr = orc.gemm_rows(W, M, N, X)
    scale = np.abs(orc.dequant_np(W).astype(np.float64)) @ np.abs(X.astype(np.float64)).T
    assert np.max(np.abs(Y.astype(np.float64) - Yr) / np.maximum(scale.T, 1e-300)) <= 2e-7


def test_gemm_multi_equals_single_and_is_deterministic(qa):
    # N = 1024 (32 blocks) keeps one K split for both launch shapes, so the
    # fused launch must reproduce the single ones bit for bit.
    M1, M2, N, T = 200, 136, 1024, 70
    rng = orc.rng_for(31, 2)
    W1, W2 = orc.gen_q4(M1, N, rng), orc.gen_q4(M2, N, rng)
    X = rng.standard_normal((T, N), dtype=np.float32)
    g = Gemm(qa, [W1, W2], [M1, M2], N, T)
    Y1, Y2 = g(X)
    Z1, Z2 = g(X)
    assert np.array_equal(Y1, Z1) and np.array_equal(Y2, Z2)
    (S1,) = Gemm(qa, [W1], [M1], N, T)(X)
    (S2,) = Gemm(qa, [W2], [M2], N, T)(X)
    assert np.array_equal(Y1, S1) and np.array_equal(Y2, S2)
    # three matrices (the Q|K|V launch of the prefill: segment boundaries
    # inside the m-tile sequence at 200 and 336 rows)
    M3 = 72
    W3 = orc.gen_q4(M3, N, rng)
    Q1, Q2, Q3 = Gemm(qa, [W1, W2, W3], [M1, M2, M3], N, T)(X)
    (S3,) = Gemm(qa, [W3], [M3], N, T)(X)
    assert np.array_equal(Q1, S1) and np.array_equal(Q2, S2) and np.array_equal(Q3, S3)


def test_gemm_two_tile_heights_match_single_launches(qa):
    """Tile heights of 256 and 192 rows, chosen per launch by a cost model of
    workgroup rounds.  Two matrices of 14336 rows at T = 512 (N = 1024: no
    K split) run rows 0..16383 in 256-row tiles and the rest in 192-row tiles
    in a second launch, the cut falling inside the second matrix; alone, each
    runs 256-row tiles.  The tile height does not change any output's
    arithmetic: every output must equal the single launches' bit for bit,
    and the oracle on sampled tokens."""
    M, N, T = 14336, 1024, 512
    rng = orc.rng_for(41, 7)
    Ws = [orc.gen_q4(M, N, rng) for _ in range(2)]
    X = rng.standard_normal((T, N), dtype=np.float32)
    Ys = Gemm(qa, Ws, [M, M], N, T)(X)
    for W, Y in zip(Ws, Ys):
        (S,) = Gemm(qa, [W], [M], N, T)(X)
        assert np.array_equal(Y, S)
    check_rows(Ws[1], M, N, X, Ys[1], [0, 300, 511])


def test_gemm_scaled_and_nonfinite_rows(qa):
    """Per-token power-of-two scaling: rows of very different magnitude, an
    all-zero row, and a row holding Inf/NaN (-> NaN outputs for that token
    only)."""
    M, N, T = 128, 512, 6
    rng = orc.rng_for(33, 3)
    W = orc.gen_q4(M, N, rng)
    X = rng.standard_normal((T, N), dtype=np.float32)
    X[1] *= np.float32(1e-30)
    X[2] *= np.float32(1e30)
    X[3] = 0.0
    X[4, 17] = np.inf
    X[5, 3] = np.nan
    (Y,) = Gemm(qa, [W], [M], N, T)(X)
    check_rows(W, M, N, X, Y, [0, 1, 2])
    assert np.all(Y[3] == 0.0)
    assert np.all(np.isnan(Y[4])) and np.all(np.isnan(Y[5]))


def test_gemm_config5_full(qa):
    """X 512x4096 against W_gate|W_up 14336x4096 (one
    launch), then 512x14336 against W_down 4096x14336.  Sampled tokens vs
    fp64/AVX2; every token vs the GPU GEMV."""
    lib = qa.lib()
    T, D, H = 512, 4096, 14336
    rng = orc.rng_for(55, 5)
    Wg, Wu, Wd = orc.gen_q4(H, D, rng), orc.gen_q4(H, D, rng), orc.gen_q4(D, H, rng)
    X = rng.standard_normal((T, D), dtype=np.float32)
    G, U = Gemm(qa, [Wg, Wu], [H, H], D, T)(X)
    Hm = rng.standard_normal((T, H), dtype=np.float32)
    (Y,) = Gemm(qa, [Wd], [D], H, T)(Hm)
    toks = [0, 1, 255, 511]
    e1, a1 = check_rows(Wg, H, D, X, G, toks)
    e2, a2 = check_rows(Wu, H, D, X, U, toks[:2])
    e3, a3 = check_rows(Wd, D, H, Hm, Y, toks)
    print(f"config 5: gate {e1:.2e} (avx2 {a1:.2e}) up {e2:.2e} (avx2 {a2:.2e}) down {e3:.2e} (avx2 {a3:.2e})")
    # every token vs the device GEMV (error bound: both within ~1e-7 of fp64)
    for W, M, N, Xs, Ys in ((Wg, H, D, X, G), (Wd, D, H, Hm, Y)):
        dW = qa.DeviceBuffer.from_numpy(np.ascontiguousarray(W))
        t = qa.q4_tensor(dW.ptr, M, N)
        dx = qa.DeviceBuffer(N * 4)
        dy = qa.DeviceBuffer(M * 4)
        ws = qa.DeviceBuffer(lib.qh_gemv_workspace_bytes(N))
        cond = (np.abs(orc.dequant_np(W).astype(np.float32)) @ np.abs(Xs).T).T  # [T, M]
        for tok in range(T):
            dx.upload(Xs[tok])
            qa.check(lib.qh_gemv_q4_f32(t.addr, dx.ptr, dy.ptr, ws.ptr, None))
            qa.check(lib.qh_device_synchronize())
            yv = dy.download(np.float32, (M,))
            d = np.abs(Ys[tok].astype(np.float64) - yv) / np.maximum(cond[tok], 1e-30)
            assert float(d.max()) <= 1e-6, tok


def test_gemm_api_errors(qa):
    lib = qa.lib()
    M, N, T = 64, 128, 4
    W = orc.gen_q4(M, N, orc.rng_for(1, 1))
    dW = qa.DeviceBuffer.from_numpy(W)
    t = qa.q4_tensor(dW.ptr, M, N)
    dX, dY = qa.DeviceBuffer(T * N * 4), qa.DeviceBuffer(T * M * 4)
    ws = qa.DeviceBuffer(lib.qh_gemm_workspace_bytes(N, T, M))
    f = lib.qh_gemm_q4_f32
    assert f(None, dX.ptr, T, dY.ptr, ws.ptr, None) == -10
    assert f(t.addr, None, T, dY.ptr, ws.ptr, None) == -10
    assert f(t.addr, dX.ptr, T, None, ws.ptr, None) == -10
    assert f(t.addr, dX.ptr + 4, T, dY.ptr, ws.ptr, None) == -13
    assert f(t.addr, dX.ptr, 0, dY.ptr, ws.ptr, None) == -15
    assert f(t.addr, dX.ptr, T, dX.ptr, ws.ptr, None) == -11
    assert f(t.addr, dX.ptr, T, dY.ptr, None, None) == -10
    # Operands that are not device memory of the needed extent are refused
    # before any launch: a host X, a Y one row short, a short workspace.
    hostX = np.zeros((T, N), np.float32)
    assert f(t.addr, hostX.ctypes.data, T, dY.ptr, ws.ptr, None) == -10
    short = qa.DeviceBuffer(T * M * 4 - 256)
    assert f(t.addr, dX.ptr, T, short.ptr, ws.ptr, None) == -10
    ws_short = qa.DeviceBuffer(lib.qh_gemm_workspace_bytes(N, T, M) - 1024)
    assert f(t.addr, dX.ptr, T, dY.ptr, ws_short.ptr, None) == -10
    bad = qa.q4_tensor(dW.ptr, M, N)
    bad.t.type = qa.Q_F32
    assert f(bad.addr, dX.ptr, T, dY.ptr, ws.ptr, None) == -14
    assert lib.qh_gemm_q4_f32_multi(None, None, 1, dX.ptr, T, ws.ptr, None) == -10
    Ws = (C.c_void_p * 4)(t.addr, t.addr, t.addr, t.addr)
    Ys = (C.c_void_p * 4)(dY.ptr, dY.ptr, dY.ptr, dY.ptr)
    assert lib.qh_gemm_q4_f32_multi(Ws, Ys, 4, dX.ptr, T, ws.ptr, None) == -15
    assert f(t.addr, dX.ptr, T, dY.ptr, ws.ptr, None) == 0
    assert lib.qh_device_synchronize() == 0


def test_gemm_activation_outliers(qa):
    """Outliers of 1e3, 1e4 and 1e5 (one channel, one column of every block,
    2/3/4/6 equal ones in one block or in every block, four of mixed sizes),
    meeting a zero weight (nibble 8) in every row, 512 rows per token.  Each
    token row: max <= 1e-5 of the condition and RMS no worse than the AVX2
    order's.  The per-token maximum over 512 rows is a tail statistic of
    both error distributions (the GEMM's RMS is 0.4-0.8x the AVX2 order's,
    and its largest row measured 1.73x the AVX2 order's largest at a 1e3
    channel outlier, once in 18,944 rows), so the maxima are compared pooled
    over all the test's rows and held to 2x.  With 1e5 outliers the row
    scale leaves elements ~1e-5 of the maximum fewer than 22 bits (fp16
    lo parts below the normal range); the RMS measured 4.3-4.9e-9 there
    against 3.4-3.9e-9 for 1e3/1e4."""
    from adversarial import CASES, Layout, apply_case, set_nibble8
    for N in (4096, 14336):
        M = 512
        rng = orc.rng_for(808, N)
        lay = Layout(N, rng)
        W = set_nibble8(orc.gen_q4(M, N, rng), lay.zero_columns())
        base = rng.standard_normal((len(CASES) + 1, N), dtype=np.float32)
        X = np.stack([base[0]] + [apply_case(base[i + 1], lay, k, n, m)
                                  for i, (k, n, m) in enumerate(CASES)])
        (Y,) = Gemm(qa, [W], [M], N, X.shape[0])(X)
        emax = amax = 0.0
        for t in range(X.shape[0]):
            y64, cond = orc.gemv_f64(W, M, N, X[t])
            cond = np.maximum(cond, 1e-300)
            e = np.abs(Y[t].astype(np.float64) - y64) / cond
            ea = np.abs(orc.gemv(W, M, N, X[t]).astype(np.float64) - y64) / cond
            assert e.max() <= 1e-5, (t, e.max())
            assert np.sqrt(np.mean(e * e)) <= np.sqrt(np.mean(ea * ea)), (t, e, ea)
            emax, amax = max(emax, float(e.max())), max(amax, float(ea.max()))
        print(f"outliers N={N}: max err/cond {emax:.3e} (avx2 order {amax:.3e})")
        assert emax <= 2.0 * amax
