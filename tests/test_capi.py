"""C-ABI of libqorus_hip.so without a GPU: the library loads, exports every
function include/*.h declares, and reproduces the reference's argument
validation order and return codes (all of which are decided before any
device work, so they run on any host).

Error-contract cases follow the reference's adversarial tests:
tests/test_matmul_adversarial.c:622-776 (misaligned, NULL, invalid N,
aliasing), tests/test_softmax_adversarial.c:114-176, the validation blocks
of src/ops/avx2/*.c, and src/core/memory.c for the memory tiers.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import qorus_amd as qa
from qorus_amd import _lib as L

REPO = Path(__file__).resolve().parent.parent
HEADERS = [REPO / "include" / "qorus.h", REPO / "include" / "qorus_hip.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:q|qh|llama)_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    assert qa.LIB_PATH.exists(), "build libqorus_hip.so first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", str(qa.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    decl = declared_functions()
    assert len(decl) >= 30
    missing = [n for n in decl if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    lib = qa.lib()
    for n in decl:
        assert hasattr(lib, n)


def declared_prototypes():
    """{name: (return kind, [parameter kinds])} from include/*.h, each type
    reduced to its ABI class: "ptr" (any pointer or handle), "i32", "u32",
    "u64", "f32", "bool", "void"."""
    scalar = {"int": "i32", "uint32_t": "u32", "uint64_t": "u64", "size_t": "u64", "float": "f32", "void": "void",
              "bool": "bool"}
    types = (REPO / "include" / "qorus_types.h").read_text()
    for enum in re.findall(r"typedef\s+enum\s*\{[^}]*\}\s*(\w+)\s*;", types):
        scalar[enum] = "i32"
    handles = {"qh_stream", "qh_event", "qh_graph"}

    def kind(decl):
        decl = re.sub(r"\b(const|Q_RESTRICT)\b", " ", decl)
        if "*" in decl:
            return "ptr"
        words = decl.split()
        base = words[0]
        if base in handles:
            return "ptr"
        return scalar[base]

    protos = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"^([A-Za-z_][\w \*]*?)\b((?:q|qh|llama)_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
            params = [p.strip() for p in m.group(3).split(",") if p.strip()]
            if params == ["void"]:
                params = []
            protos[m.group(2)] = (kind(m.group(1)), [kind(p) for p in params])
    return protos


def ctypes_kind(t):
    if t is None:
        return "void"
    if t in (C.c_void_p, C.c_char_p) or issubclass(t, C._Pointer):
        return "ptr"
    if t is C.c_float:
        return "f32"
    if t is C.c_bool:
        return "bool"
    if t in (C.c_int, C.c_int32):
        return "i32"
    if t in (C.c_uint32, C.c_uint):
        return "u32"
    if t in (C.c_uint64, C.c_size_t, C.c_ulonglong, C.c_ulong):
        return "u64"
    raise AssertionError(f"unmapped ctypes type {t}")


def test_ctypes_bindings_match_declarations():
    """Every ctypes binding in qorus_amd._lib has the argument and return
    classes of its declaration.  A binding that passes a pointer through a
    32-bit integer slot truncates the device address, and the kernel then
    writes to an unmapped one."""
    protos = declared_prototypes()
    assert len(protos) >= 40
    lib = qa.lib()
    checked = 0
    for name, (ret, params) in protos.items():
        fn = getattr(lib, name)
        if fn.argtypes is None:
            continue
        got = [ctypes_kind(t) for t in fn.argtypes]
        assert got == params, f"{name}: bound {got}, declared {params}"
        assert ctypes_kind(fn.restype) == ret, f"{name}: returns {fn.restype}, declared {ret}"
        checked += 1
    assert checked >= 40


def test_strerror_table():
    lib = qa.lib()
    assert lib.q_strerror(0) == b"Success"
    for code in range(-15, 1):
        assert lib.q_strerror(code)
    assert lib.q_strerror(-99) == b"Unknown error"


def aligned(n, dtype=np.float32, off=0):
    a = np.zeros(n + 64, dtype=dtype)
    base = (-a.ctypes.data) % 64 // a.itemsize
    return a[base + off: base + off + n]


def test_gemv_validation_order():
    lib = qa.lib()
    W = aligned(4 * 4 * 20, np.uint8)
    x = aligned(128)
    y = aligned(4)
    t = qa.q4_tensor(W.ctypes.data, 4, 128)
    g = lambda tt, xx, yy: lib.q_gemv_q4_f32_avx2(tt, xx, yy)
    assert g(None, x.ctypes.data, y.ctypes.data) == L.Q_ERR_INVALID_ARG
    assert g(t.addr, None, y.ctypes.data) == L.Q_ERR_INVALID_ARG
    assert g(t.addr, x.ctypes.data, None) == L.Q_ERR_INVALID_ARG
    assert g(t.addr, x.ctypes.data + 4, y.ctypes.data) == L.Q_ERR_MISALIGNED
    assert g(t.addr, x.ctypes.data, y.ctypes.data + 4) == L.Q_ERR_MISALIGNED
    assert g(t.addr, x.ctypes.data, x.ctypes.data) == L.Q_ERR_ALIASING
    for M, N in ((0, 128), (4, 0), (4, 100)):
        tt = qa.q4_tensor(W.ctypes.data, M, N, nb0=80)
        assert g(tt.addr, x.ctypes.data, y.ctypes.data) == L.Q_ERR_INVALID_SIZE
    tf = qa.q4_tensor(W.ctypes.data, 4, 128)
    tf.t.type = qa.Q_F32
    assert g(tf.addr, x.ctypes.data, y.ctypes.data) == L.Q_ERR_INVALID_DTYPE
    big = qa.q4_tensor(W.ctypes.data, 0x10000000, 32 * 64)
    assert g(big.addr, x.ctypes.data, y.ctypes.data) == L.Q_ERR_OVERFLOW
    # nb[0] left 0 (as the reference's adversarial tests build it) -> INVALID_ARG
    z = qa.q4_tensor(W.ctypes.data, 4, 128, nb0=0)
    assert g(z.addr, x.ctypes.data, y.ctypes.data) == L.Q_ERR_INVALID_ARG
    # device entry points share the validation
    assert lib.qh_gemv_q4_f32(z.addr, x.ctypes.data, y.ctypes.data, None, None) == L.Q_ERR_INVALID_ARG
    assert lib.qh_gemv_q4_f32(t.addr, x.ctypes.data, x.ctypes.data, None, None) == L.Q_ERR_ALIASING


def test_vector_op_validation():
    lib = qa.lib()
    a, b, o = aligned(64), aligned(64), aligned(64)
    p = lambda v: v.ctypes.data
    assert lib.q_rmsnorm_f32_avx2(None, p(b), p(o), 64, 1e-5) == L.Q_ERR_INVALID_ARG
    assert lib.q_rmsnorm_f32_avx2(p(a) + 4, p(b), p(o), 64, 1e-5) == L.Q_ERR_MISALIGNED
    assert lib.q_rmsnorm_f32_avx2(p(a), p(b), p(o), 0, 1e-5) == L.Q_ERR_INVALID_SIZE
    assert lib.q_rmsnorm_f32_avx2(p(a), p(b), p(o), 12, 1e-5) == L.Q_ERR_INVALID_SIZE
    assert lib.q_rope_f32_avx2(p(a), None, p(b), p(o), 64) == L.Q_ERR_INVALID_ARG
    assert lib.q_rope_f32_avx2(p(a), p(a), p(b) + 8, p(o), 64) == L.Q_ERR_MISALIGNED
    assert lib.q_rope_f32_avx2(p(a), p(a), p(b), p(o), 6) == L.Q_ERR_INVALID_SIZE
    assert lib.q_silu_f32_avx2(None, p(o), 8) == L.Q_ERR_INVALID_ARG
    assert lib.q_silu_f32_avx2(p(a), p(o), 0) == L.Q_ERR_INVALID_SIZE
    assert lib.q_silu_f32_avx2(p(a) + 4, p(o), 8) == L.Q_ERR_MISALIGNED
    assert lib.q_softmax_f32_avx2(p(a), None, 8) == L.Q_ERR_INVALID_ARG
    assert lib.q_softmax_f32_avx2(p(a), p(o), 0) == L.Q_ERR_INVALID_SIZE
    assert lib.q_softmax_f32_avx2(p(a), p(o) + 4, 16) == L.Q_ERR_MISALIGNED
    ta, tb, to = qa.f32_tensor(p(a), 64), qa.f32_tensor(p(b), 64), qa.f32_tensor(p(o), 64)
    assert lib.q_add_f32_avx2(None, tb.addr, to.addr) == L.Q_ERR_INVALID_ARG
    t2 = qa.f32_tensor(p(a), 64)
    t2.t.ne[1] = 2
    assert lib.q_add_f32_avx2(t2.addr, tb.addr, to.addr) == L.Q_ERR_INVALID_SIZE
    t3 = qa.f32_tensor(p(b), 32)
    assert lib.q_mul_f32_avx2(ta.addr, t3.addr, to.addr) == L.Q_ERR_INVALID_SIZE
    t4 = qa.f32_tensor(p(a), 64)
    t4.t.type = qa.Q_Q4_0
    assert lib.q_mul_f32_avx2(t4.addr, tb.addr, to.addr) == L.Q_ERR_INVALID_DTYPE
    t5 = qa.f32_tensor(p(a), 64)
    t5.t.nb[0] = 4
    assert lib.q_add_f32_avx2(t5.addr, tb.addr, to.addr) == L.Q_ERR_INVALID_SIZE
    t6 = qa.f32_tensor(p(a) + 4, 64)
    assert lib.q_add_f32_avx2(t6.addr, tb.addr, to.addr) == L.Q_ERR_MISALIGNED


class Ctx(C.Structure):
    _fields_ = [("weights_mmap", C.c_void_p), ("weights_size", C.c_size_t), ("header", C.c_void_p),
                ("kv_buffer", C.c_void_p), ("kv_size", C.c_size_t),
                ("scratch_buffer", C.c_void_p), ("scratch_size", C.c_size_t),
                ("scratch_head", C.c_size_t), ("scratch_base_offset", C.c_size_t)]


def test_context_layout():
    assert C.sizeof(Ctx) == 72


def test_host_arena_semantics():
    lib = qa.lib()
    ctx = Ctx()
    assert lib.q_alloc_arena(C.byref(ctx), 1000) == 0
    assert ctx.scratch_size == 1024
    assert lib.q_alloc_arena(C.byref(ctx), 10) == L.Q_ERR_INVALID_ARG  # leak guard
    p1 = lib.q_arena_alloc(C.byref(ctx), 1)
    p2 = lib.q_arena_alloc(C.byref(ctx), 65)
    assert p1 % 64 == 0 and p2 - p1 == 64 and ctx.scratch_head == 192
    ctx.scratch_base_offset = 64
    lib.q_arena_reset(C.byref(ctx))
    assert ctx.scratch_head == 64
    assert lib.q_arena_alloc(C.byref(ctx), 4096) is None  # OOM -> NULL
    assert lib.q_arena_alloc(None, 8) is None
    lib.q_free_memory(C.byref(ctx))
    assert ctx.scratch_buffer is None and ctx.scratch_size == 0


def test_init_memory_file_errors(tmp_path):
    lib = qa.lib()
    ctx = Ctx()
    assert lib.q_init_memory(None, b"x") == L.Q_ERR_INVALID_ARG
    assert lib.q_init_memory(C.byref(ctx), str(tmp_path / "missing").encode()) == L.Q_ERR_FILE_OPEN
    small = tmp_path / "small.qorus"
    small.write_bytes(b"\0" * 10)
    assert lib.q_init_memory(C.byref(ctx), str(small).encode()) == L.Q_ERR_FILE_TOO_SMALL
    bad = tmp_path / "bad.qorus"
    bad.write_bytes(b"\1" * 128)
    assert lib.q_init_memory_ex(C.byref(ctx), str(bad).encode(), 1) == L.Q_ERR_INVALID_MAGIC
    assert ctx.weights_mmap is None


def test_model_file_layout_agrees_with_oracle(tmp_path):
    from oracle import oracle as orc
    h = qa.QorusHeader(vocab=100, dim=64, hidden=96, n_layers=2, n_heads=4, n_kv=2, max_seq=16)
    lay = qa.model_layout(h)
    rng = orc.rng_for(5)

    def get(name, kind, shape):
        if kind == "f32":
            return rng.standard_normal(shape, dtype=np.float32)
        return orc.gen_q4(shape[0], shape[1], rng)

    path = tmp_path / "m.qorus"
    size = qa.write_qorus_v3(path, h, get)
    blob = np.fromfile(path, dtype=np.uint8)
    assert size == lay["_size"] == blob.size
    hd = orc.parse_header(blob)
    assert hd["version"] == 3 and hd["dim"] == 64 and hd["n_kv"] == 2
    olay = orc.model_layout(hd)
    for k, v in lay.items():
        assert olay[k] == v, k


def test_matmul_f32_validation_order():
    """q_matmul_f32_avx2 error codes in the reference's order
    (matmul_fp32.c:64-285); all of these return before any device work."""
    import ctypes as C
    import numpy as np
    from oracle import oracle as orc
    from qorus_amd._lib import _AlignedTensor
    from qorus_amd.model import QContext
    lib = L.lib()
    A = orc.aligned_empty((4, 64), np.float32)
    B = orc.aligned_empty((64, 8), np.float32)
    Cm = orc.aligned_empty((4, 8), np.float32)

    def T(arr, ne0, ne1, nb0, nb1=4, dtype=None, off=0):
        return _AlignedTensor(arr.ctypes.data + off, (ne0, ne1, 1, 1), (nb0, nb1, 4, 4),
                              L.Q_F32 if dtype is None else dtype)

    ctx = QContext()
    ta, tb, tc = T(A, 4, 64, 256), T(B, 64, 8, 32), T(Cm, 4, 8, 32)
    f = lambda a, b, c, x: lib.q_matmul_f32_avx2(a.addr if a else None, b.addr if b else None,
                                                 c.addr if c else None, C.byref(x) if x is not None else None)
    assert f(None, tb, tc, ctx) == -10
    assert f(ta, tb, tc, None) == -10
    assert f(T(A, 0, 64, 256), tb, tc, ctx) == -15          # M == 0
    assert f(ta, T(B, 63, 8, 32), tc, ctx) == -15           # B->ne[0] != K
    assert f(ta, tb, T(Cm, 4, 7, 32), ctx) == -15           # C->ne[1] != N
    assert f(T(A, 4, 64, 256, off=4), tb, tc, ctx) == -13   # A->data misaligned with aligned stride
    assert f(ta, T(B, 64, 8, 32, dtype=L.Q_Q4_0), tc, ctx) == -14
    assert f(T(A, 4, 64, 128), tb, tc, ctx) == -15          # A stride < K
    assert f(ta, T(B, 64, 8, 16), tc, ctx) == -15           # B stride < N
    assert f(ta, tb, T(Cm, 4, 8, 16), ctx) == -15           # C stride < N
    assert f(ta, tb, tc, ctx) == -8                         # no arena for the transpose buffer
    # a misaligned A with an unaligned stride is accepted by validation
    # (then the transpose buffer is the first failure here)
    assert f(T(A, 4, 60, 244, off=4), T(B, 60, 8, 32), tc, ctx) == -8
