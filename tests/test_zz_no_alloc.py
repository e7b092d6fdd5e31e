"""The allocation-free LM-head entry point, qh_gemv_q4_f32_softmax_argmax_noalloc,
against the workspace form qh_gemv_q4_f32_softmax_argmax through the C-ABI.

Both run the same kernels, so the bar is bit-identity of logits and
probabilities and the same argmax index.  The no-alloc calls run back to
back, each smaller than the one before, so every call after the first finds
the previous call's partials in the shared scratch array.  The shapes cover
the three launch forms: the GEMV that leaves argmax partials (2048 < N <=
4096, M >= 16384), the multi-workgroup softmax after a plain GEMV (N = 8192),
and the one-workgroup kernels (M < 16384).
"""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [(128256, 4096), (40000, 8192), (3000, 1024)]


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


class LmHead:
    def __init__(self, qa, M, N, seed):
        self.qa, self.M, self.N = qa, M, N
        rng = orc.rng_for(seed, M, N)
        self.dW = qa.DeviceBuffer.from_numpy(orc.gen_q4(M, N, rng))
        self.dx = qa.DeviceBuffer.from_numpy(orc.gen_f32(N, rng))
        self.t = qa.q4_tensor(self.dW.ptr, M, N)
        self.logits = qa.DeviceBuffer(M * 4)
        self.probs = qa.DeviceBuffer(M * 4)
        self.idx = qa.DeviceBuffer(256)

    def outputs(self):
        return (self.logits.download(np.float32, (self.M,)), self.probs.download(np.float32, (self.M,)),
                int(self.idx.download(np.uint32, (1,))[0]))


def test_noalloc_equals_workspace_form(qa):
    lib = qa.lib()
    heads = [LmHead(qa, M, N, 900 + i) for i, (M, N) in enumerate(CASES)]
    want = []
    for h in heads:
        ws = qa.DeviceBuffer(lib.qh_gemv_softmax_workspace_bytes(h.M))
        qa.check(lib.qh_gemv_q4_f32_softmax_argmax(h.t.addr, h.dx.ptr, h.logits.ptr, h.probs.ptr, h.idx.ptr,
                                                   ws.ptr, None), "workspace form")
        qa.check(lib.qh_device_synchronize())
        want.append(h.outputs())
        h.logits.zero(); h.probs.zero(); h.idx.zero()
        qa.check(lib.qh_device_synchronize())
    # The no-alloc calls back to back (largest first), then compared.
    for h in heads:
        qa.check(lib.qh_gemv_q4_f32_softmax_argmax_noalloc(h.t.addr, h.dx.ptr, h.logits.ptr, h.probs.ptr,
                                                           h.idx.ptr, None), "noalloc form")
    qa.check(lib.qh_device_synchronize())
    for h, (lw, pw, iw) in zip(heads, want):
        lg, pg, ig = h.outputs()
        assert np.array_equal(_bits(lg), _bits(lw)), (h.M, h.N)
        assert np.array_equal(_bits(pg), _bits(pw)), (h.M, h.N)
        assert ig == iw == int(np.argmax(lw)), (h.M, h.N, ig, iw)


def test_noalloc_under_graph_capture(qa):
    """The no-alloc calls captured into a HIP graph (thread-local capture
    mode, which refuses device allocations), then the graph replayed three
    times with eager clears of the outputs in between: every replay gives
    the workspace form's bits."""
    lib = qa.lib()
    heads = [LmHead(qa, M, N, 950 + i) for i, (M, N) in enumerate(CASES)]
    want = []
    for h in heads:
        ws = qa.DeviceBuffer(lib.qh_gemv_softmax_workspace_bytes(h.M))
        qa.check(lib.qh_gemv_q4_f32_softmax_argmax(h.t.addr, h.dx.ptr, h.logits.ptr, h.probs.ptr, h.idx.ptr,
                                                   ws.ptr, None), "workspace form")
        qa.check(lib.qh_device_synchronize())
        want.append(h.outputs())
    st = qa.Stream()
    qa.check(lib.qh_stream_begin_capture(st.handle), "begin capture")
    for h in heads:
        rc = lib.qh_gemv_q4_f32_softmax_argmax_noalloc(h.t.addr, h.dx.ptr, h.logits.ptr, h.probs.ptr,
                                                       h.idx.ptr, st.handle)
        if rc != 0:
            import ctypes as C
            g = C.c_void_p()
            lib.qh_stream_end_capture(st.handle, C.byref(g))
            qa.check(rc, "noalloc under capture")
    import ctypes as C
    graph = C.c_void_p()
    qa.check(lib.qh_stream_end_capture(st.handle, C.byref(graph)), "end capture")
    try:
        for rep in range(3):
            for h in heads:
                h.logits.zero(); h.probs.zero(); h.idx.zero()
            qa.check(lib.qh_device_synchronize())
            qa.check(lib.qh_graph_launch(graph.value, st.handle), "replay")
            st.sync()
            for h, (lw, pw, iw) in zip(heads, want):
                lg, pg, ig = h.outputs()
                assert np.array_equal(_bits(lg), _bits(lw)), (rep, h.M, h.N)
                assert np.array_equal(_bits(pg), _bits(pw)), (rep, h.M, h.N)
                assert ig == iw, (rep, h.M, h.N)
    finally:
        lib.qh_graph_destroy(graph.value)


def test_noalloc_errors(qa):
    lib = qa.lib()
    f = lib.qh_gemv_q4_f32_softmax_argmax_noalloc
    h = LmHead(qa, 64, 16416, 7)  # N above 16384
    assert f(h.t.addr, h.dx.ptr, h.logits.ptr, h.probs.ptr, h.idx.ptr, None) == -15
    g = LmHead(qa, 64, 256, 8)
    assert f(g.t.addr, g.dx.ptr, g.logits.ptr, None, g.idx.ptr, None) == -10
    assert f(g.t.addr, g.dx.ptr, g.logits.ptr, g.probs.ptr, None, None) == -10
    assert f(g.t.addr, g.dx.ptr, g.logits.ptr, g.logits.ptr, g.idx.ptr, None) == -11
    # operands that are not device memory of the required extent: refused
    hx = orc.aligned_copy(orc.gen_f32(256, orc.rng_for(9)))
    assert f(g.t.addr, hx.ctypes.data, g.logits.ptr, g.probs.ptr, g.idx.ptr, None) == -10
    short = qa.DeviceBuffer(32 * 4)
    assert f(g.t.addr, g.dx.ptr, g.logits.ptr, short.ptr, g.idx.ptr, None) == -10
    hw = orc.aligned_copy(orc.gen_q4(64, 256, orc.rng_for(10)).reshape(-1))
    th = qa.q4_tensor(hw.ctypes.data, 64, 256)
    assert f(th.addr, g.dx.ptr, g.logits.ptr, g.probs.ptr, g.idx.ptr, None) == -10
    assert f(g.t.addr, g.dx.ptr, g.logits.ptr, g.probs.ptr, g.idx.ptr, None) == 0
    assert lib.qh_device_synchronize() == 0
