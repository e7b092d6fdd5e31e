"""ctypes front-end of the CPU oracle (test infrastructure only).

Loads oracle/build/liboracle.so (this repo's plain-C restatement of the
reference ops) and, when it was built, oracle/_ref/libqorus_ref.so (the
reference's own hot-path C sources compiled in place by `make -C oracle ref`).
Also holds the seeded input generators shared by the tests and bench.py, and
an independent parser of the .qorus v3 layout used to feed or_decode_step.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
_LIB = ORACLE_DIR / "build" / "liboracle.so"
_REF = ORACLE_DIR / "_ref" / "libqorus_ref.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")

Q_OK = 0
Q_Q4_0 = 2
Q_F32 = 0


def aligned_empty(shape, dtype, align: int = 64) -> np.ndarray:
    """Uninitialised C-contiguous array whose data pointer is `align`-aligned."""
    dtype = np.dtype(dtype)
    n = int(np.prod(shape)) if shape != () else 1
    raw = np.empty(n * dtype.itemsize + align, dtype=np.uint8)
    off = (-raw.ctypes.data) % align
    return raw[off: off + n * dtype.itemsize].view(dtype).reshape(shape)


def aligned_copy(a: np.ndarray, align: int = 64) -> np.ndarray:
    out = aligned_empty(a.shape, a.dtype, align)
    out[...] = a
    return out


class QTensor(C.Structure):
    """q_tensor (reference include/qorus_types.h:205-213), 128 bytes."""
    _fields_ = [
        ("data", C.c_void_p),
        ("scales", C.c_void_p),
        ("ne", C.c_uint32 * 4),
        ("nb", C.c_size_t * 4),
        ("type", C.c_int),
        ("name", C.c_char * 32),
        ("_pad", C.c_uint8 * 28),
    ]


assert C.sizeof(QTensor) == 128


def make_tensor(data_ptr: int, ne, nb, dtype: int):
    """A q_tensor living in 64-byte aligned memory (the type is aligned(64)).
    Returns (tensor, keepalive)."""
    buf = aligned_empty((128,), np.uint8, 64)
    buf[:] = 0
    t = QTensor.from_buffer(buf)
    t.data = data_ptr
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    t.type = dtype
    return t, buf


def q4_tensor(ptr: int, M: int, N: int):
    """Q4_0 [M, N] view with the strides of reference model.c:258-273."""
    rb = N // 32 * 20
    return make_tensor(ptr, (M, N, 1, 1), (rb, 20, 20, 20), Q_Q4_0)


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (the generator BASELINE's configs describe):
# nibbles uniform 0..15, scale = |N(0,1)| * 0.02 (as float32), x ~ N(0,1).
# ---------------------------------------------------------------------------

def rng_for(seed: int, *stream) -> np.random.Generator:
    return np.random.default_rng([int(seed)] + [int(s) for s in stream])


def gen_q4(M: int, N: int, rng: np.random.Generator) -> np.ndarray:
    """Q4_0 matrix as uint8 [M, N/32*20] (AoS 20-byte blocks)."""
    assert N % 32 == 0
    nblk = N // 32
    blocks = np.empty((M, nblk, 20), dtype=np.uint8)
    blocks[:, :, :16] = rng.integers(0, 256, size=(M, nblk, 16), dtype=np.uint8)
    sc = (np.abs(rng.standard_normal((M, nblk), dtype=np.float32)) * np.float32(0.02)).astype(np.float32)
    blocks[:, :, 16:] = sc.view(np.uint8).reshape(M, nblk, 4)
    return blocks.reshape(M, nblk * 20)


def gen_f32(n, rng: np.random.Generator) -> np.ndarray:
    return rng.standard_normal(n, dtype=np.float32)


def q4_scales(W: np.ndarray) -> np.ndarray:
    M = W.shape[0]
    return W.reshape(M, -1, 20)[:, :, 16:].copy().view(np.float32).reshape(M, -1)


def q4_nibbles(W: np.ndarray) -> np.ndarray:
    """int nibble per element, [M, N] in element order."""
    M = W.shape[0]
    qs = W.reshape(M, -1, 20)[:, :, :16]
    lo = qs & 0x0F
    hi = qs >> 4
    out = np.empty(qs.shape[:2] + (32,), dtype=np.int32)
    out[:, :, 0::2] = lo
    out[:, :, 1::2] = hi
    return out.reshape(M, -1)


def dequant_np(W: np.ndarray) -> np.ndarray:
    """Closed form (q - 8) * s in float64 (independent of the C oracle)."""
    M = W.shape[0]
    q = q4_nibbles(W).astype(np.float64)
    s = np.repeat(q4_scales(W).astype(np.float64), 32, axis=1)
    return ((q - 8.0) * s).reshape(M, -1)


# ---------------------------------------------------------------------------
# Library bindings
# ---------------------------------------------------------------------------

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            raise RuntimeError(f"oracle not built: {_LIB} (run `make -C oracle`)")
        L = C.CDLL(str(_LIB))
        L.or_dequant_block.argtypes = [_u8p, _f32p]
        L.or_dequant_blocks.argtypes = [_u8p, C.c_uint64, _f32p]
        L.or_set_threads.argtypes = [C.c_int]
        L.or_set_threads.restype = None
        L.or_gemv_q4.argtypes = [_u8p, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.or_gemv_q4_rows.argtypes = [_u8p, C.c_uint32, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.or_gemv_q4_f64.argtypes = [_u8p, C.c_uint32, C.c_uint32, _f32p, _f64p, _f64p]
        L.or_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_uint32, C.c_float]
        L.or_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_uint32]
        L.or_rope_tables.argtypes = [C.c_float, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.or_exp_approx.argtypes = [C.c_float]
        L.or_exp_approx.restype = C.c_float
        L.or_silu.argtypes = [_f32p, _f32p, C.c_uint32]
        L.or_softmax.argtypes = [_f32p, _f32p, C.c_uint32]
        L.or_argmax.argtypes = [_f32p, C.c_uint32]
        L.or_argmax.restype = C.c_uint32
        L.or_add.argtypes = [_f32p, _f32p, _f32p, C.c_uint32]
        L.or_mul.argtypes = [_f32p, _f32p, _f32p, C.c_uint32]
        L.or_causal_mask.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_float]
        L.or_dot_f32.argtypes = [_f32p, _f32p, C.c_uint32]
        L.or_dot_f32.restype = C.c_float
        L.or_matmul_f32.argtypes = [_f32p, _f32p, _f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.or_attention_decode.argtypes = [_f32p, _f32p, _f32p, C.c_uint32, C.c_uint32,
                                          C.c_uint32, C.c_uint32, C.c_uint32]
        L.or_gemm_q4_rows.argtypes = [_u8p, C.c_uint32, C.c_uint32, _f32p, C.c_uint32, _f32p]
        L.or_decode_step.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
        L.or_decode_step.restype = C.c_uint32
        L.or_sample_token.argtypes = [C.c_void_p, C.c_uint32, C.c_float, C.c_uint32, C.c_float, C.c_int, C.c_int,
                                      C.POINTER(C.c_uint64)]
        L.or_sample_token.restype = C.c_uint32
        _lib = L
    return _lib


class QContext(C.Structure):
    """q_context (reference include/qorus_types.h:216-231), 72 bytes."""
    _fields_ = [("weights_mmap", C.c_void_p), ("weights_size", C.c_size_t), ("header", C.c_void_p),
                ("kv_buffer", C.c_void_p), ("kv_size", C.c_size_t),
                ("scratch_buffer", C.c_void_p), ("scratch_size", C.c_size_t),
                ("scratch_head", C.c_size_t), ("scratch_base_offset", C.c_size_t)]


RNG_SEED = 123456789  # the reference sampler's initial xorshift64* state (main.c:949)


def sample_token(logits: np.ndarray, temperature: float, top_k: int, top_p: float, state: C.c_uint64,
                 nucleus_all: bool = False) -> int:
    """or_sample_token on a float32 array (its data address decides the
    reference's aligned temperature path); state is advanced."""
    assert logits.dtype == np.float32 and logits.flags.c_contiguous
    aligned = int(logits.ctypes.data % 32 == 0)
    return int(lib().or_sample_token(logits.ctypes.data, logits.size, temperature, top_k, top_p, aligned,
                                     int(nucleus_all), C.byref(state)))


class RefSampler:
    """A private copy of oracle/_ref's library (its own thread-local RNG
    state, starting at RNG_SEED) with an arena-backed q_context, calling
    the reference's own q_sample_token."""

    def __init__(self, tmp_dir, arena_bytes: int = 64 << 20):
        import shutil
        import uuid
        # a new file per instance: copying over a library that is still
        # mapped would corrupt it
        path = Path(tmp_dir) / f"libqorus_ref_{uuid.uuid4().hex}.so"
        shutil.copy(_REF, path)
        R = C.CDLL(str(path))
        R.q_alloc_arena.argtypes = [C.c_void_p, C.c_size_t]
        R.q_alloc_arena.restype = C.c_int
        R.q_arena_reset.argtypes = [C.c_void_p]
        R.q_arena_reset.restype = None
        R.q_free_memory.argtypes = [C.c_void_p]
        R.q_free_memory.restype = None
        R.q_sample_token.argtypes = [C.c_void_p, C.c_uint32, C.c_float, C.c_uint32, C.c_float, C.c_void_p,
                                     C.c_void_p]
        R.q_sample_token.restype = C.c_int
        self.R = R
        self.ctx = QContext()
        if arena_bytes:
            assert R.q_alloc_arena(C.byref(self.ctx), arena_bytes) == Q_OK

    def sample(self, logits: np.ndarray, temperature: float, top_k: int, top_p: float, reset: bool = True):
        """(return code, token); the arena is reset first unless reset=False."""
        if reset and self.ctx.scratch_buffer:
            self.R.q_arena_reset(C.byref(self.ctx))
        tok = C.c_uint32(0xFFFFFFFF)
        ctx = C.byref(self.ctx) if self.ctx.scratch_buffer else None
        rc = self.R.q_sample_token(logits.ctypes.data, logits.size, temperature, top_k, top_p, C.byref(tok), ctx)
        return rc, tok.value

    def close(self):
        self.R.q_free_memory(C.byref(self.ctx))


def ref_available() -> bool:
    return _REF.exists()


def ref():
    """The reference's own compiled hot path (oracle/_ref), or None."""
    global _ref
    if _ref is None and _REF.exists():
        R = C.CDLL(str(_REF))
        R.q_dequantize_q4_0_block_avx2_public.argtypes = [C.c_void_p, C.c_void_p]
        R.q_dequantize_q4_0_block_avx2_public.restype = None
        R.q_gemv_q4_f32_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        R.q_gemv_q4_f32_avx2.restype = C.c_int
        R.q_rmsnorm_f32_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_float]
        R.q_rmsnorm_f32_avx2.restype = C.c_int
        R.q_rope_f32_avx2.argtypes = [C.c_void_p] * 4 + [C.c_uint32]
        R.q_rope_f32_avx2.restype = C.c_int
        R.q_silu_f32_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
        R.q_silu_f32_avx2.restype = C.c_int
        R.q_softmax_f32_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
        R.q_softmax_f32_avx2.restype = C.c_int
        R.q_add_f32_avx2.argtypes = [C.c_void_p] * 3
        R.q_add_f32_avx2.restype = C.c_int
        R.q_mul_f32_avx2.argtypes = [C.c_void_p] * 3
        R.q_mul_f32_avx2.restype = C.c_int
        R.q_matmul_f32_avx2.argtypes = [C.c_void_p] * 4
        R.q_matmul_f32_avx2.restype = C.c_int
        R.q_causal_mask_f32_avx2.argtypes = [C.c_void_p, C.c_float]
        R.q_causal_mask_f32_avx2.restype = C.c_int
        R.q_alloc_arena.argtypes = [C.c_void_p, C.c_size_t]
        R.q_alloc_arena.restype = C.c_int
        R.q_free_memory.argtypes = [C.c_void_p]
        R.q_free_memory.restype = None
        _ref = R
    return _ref


# ---------------------------------------------------------------------------
# Oracle wrappers (numpy in, numpy out)
# ---------------------------------------------------------------------------

def set_threads(n: int) -> None:
    """Threads for the oracle's GEMV rows and attention heads (1 by
    default; any count gives the same bits)."""
    lib().or_set_threads(int(n))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def dequant(W: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    nb = W.size // 20
    out = np.empty(nb * 32, dtype=np.float32)
    lib().or_dequant_blocks(W.reshape(-1), nb, out)
    return out


def gemv(W: np.ndarray, M: int, N: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(M, dtype=np.float32)
    lib().or_gemv_q4(np.ascontiguousarray(W).reshape(-1), M, N, f32(x), y)
    return y


def gemv_rows(W: np.ndarray, r0: int, r1: int, N: int, x: np.ndarray, y: np.ndarray):
    lib().or_gemv_q4_rows(np.ascontiguousarray(W).reshape(-1), r0, r1, N, f32(x), y)


def gemv_f64(W: np.ndarray, M: int, N: int, x: np.ndarray):
    y = np.empty(M, dtype=np.float64)
    c = np.empty(M, dtype=np.float64)
    lib().or_gemv_q4_f64(np.ascontiguousarray(W).reshape(-1), M, N, f32(x), y, c)
    return y, c


def rmsnorm(x, w, eps=1e-5):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().or_rmsnorm(x, w, y, x.size, eps)
    return y


def rope(x, c, s):
    x = f32(x)
    y = np.empty_like(x)
    lib().or_rope(x, f32(c), f32(s), y, x.size)
    return y


def rope_tables(base: float, head_dim: int, pos: int):
    c = np.empty(head_dim, dtype=np.float32)
    s = np.empty(head_dim, dtype=np.float32)
    lib().or_rope_tables(base, head_dim, pos, c, s)
    return c, s


def exp_approx(x: float) -> float:
    return lib().or_exp_approx(x)


def silu(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().or_silu(x, y, x.size)
    return y


def softmax(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().or_softmax(x, y, x.size)
    return y


def argmax(x) -> int:
    x = f32(x)
    return int(lib().or_argmax(x, x.size))


def add(a, b):
    a, b = f32(a), f32(b)
    o = np.empty_like(a)
    lib().or_add(a, b, o, a.size)
    return o


def mul(a, b):
    a, b = f32(a), f32(b)
    o = np.empty_like(a)
    lib().or_mul(a, b, o, a.size)
    return o


def causal_mask(m: np.ndarray, n: int, v: float) -> np.ndarray:
    """or_causal_mask on a copy of m [n][ld] (row stride ld = m.shape[1])."""
    o = np.ascontiguousarray(m, dtype=np.float32).copy()
    lib().or_causal_mask(o.reshape(-1), n, o.shape[1], v)
    return o


def dot_f32(a, b) -> float:
    a, b = f32(a), f32(b)
    return float(lib().or_dot_f32(a, b, a.size))


def matmul_f32(A, B):
    A, B = f32(A), f32(B)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    Cm = np.empty((M, N), dtype=np.float32)
    lib().or_matmul_f32(A, B, Cm, M, K, N)
    return Cm


def attention_decode(q, kv_layer, n_heads, n_kv, head_dim, max_seq, pos):
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().or_attention_decode(f32(q).reshape(-1), f32(kv_layer).reshape(-1), out,
                              n_heads, n_kv, head_dim, max_seq, pos)
    return out


def gemm_rows(W, M, N, X):
    X = f32(X)
    T = X.shape[0]
    Y = np.empty((T, M), dtype=np.float32)
    lib().or_gemm_q4_rows(np.ascontiguousarray(W).reshape(-1), M, N, X.reshape(-1), T, Y.reshape(-1))
    return Y


# ---------------------------------------------------------------------------
# Reference (oracle/_ref) wrappers
# ---------------------------------------------------------------------------

def ref_gemv(W: np.ndarray, M: int, N: int, x: np.ndarray):
    """Returns (code, y) from the reference's q_gemv_q4_f32_avx2."""
    R = ref()
    Wa = aligned_copy(np.ascontiguousarray(W).reshape(-1))
    xa = aligned_copy(f32(x))
    ya = aligned_empty((M,), np.float32)
    t, keep = q4_tensor(Wa.ctypes.data, M, N)
    rc = R.q_gemv_q4_f32_avx2(C.addressof(t), xa.ctypes.data, ya.ctypes.data)
    return rc, ya.copy()


def ref_dequant_block(blk: np.ndarray) -> np.ndarray:
    R = ref()
    b = aligned_copy(np.ascontiguousarray(blk, dtype=np.uint8).reshape(20))
    out = aligned_empty((32,), np.float32)
    R.q_dequantize_q4_0_block_avx2_public(b.ctypes.data, out.ctypes.data)
    return out.copy()


def _ref_vec(fn, *arrays, n_out, extra=()):
    ins = [aligned_copy(f32(a)) for a in arrays]
    out = aligned_empty((n_out,), np.float32)
    rc = fn(*[a.ctypes.data for a in ins], out.ctypes.data, *extra)
    return rc, out.copy()


def ref_rmsnorm(x, w, eps=1e-5):
    x = f32(x)
    return _ref_vec(ref().q_rmsnorm_f32_avx2, x, w, n_out=x.size, extra=(x.size, eps))


def ref_rope(x, c, s):
    x = f32(x)
    return _ref_vec(ref().q_rope_f32_avx2, x, c, s, n_out=x.size, extra=(x.size,))


def ref_silu(x):
    x = f32(x)
    return _ref_vec(ref().q_silu_f32_avx2, x, n_out=x.size, extra=(x.size,))


def ref_softmax(x):
    x = f32(x)
    return _ref_vec(ref().q_softmax_f32_avx2, x, n_out=x.size, extra=(x.size,))


def _vec_tensor(arr):
    n = arr.size
    return make_tensor(arr.ctypes.data, (n, 1, 1, 1), (n * 4, 4, 4, 4), Q_F32)


def ref_binary(name, a, b):
    fn = getattr(ref(), name)
    aa, bb = aligned_copy(f32(a)), aligned_copy(f32(b))
    oo = aligned_empty((aa.size,), np.float32)
    ta, ka = _vec_tensor(aa)
    tb, kb = _vec_tensor(bb)
    to, ko = _vec_tensor(oo)
    rc = fn(C.addressof(ta), C.addressof(tb), C.addressof(to))
    return rc, oo.copy()


class _RefCtx(C.Structure):
    _fields_ = [("weights_mmap", C.c_void_p), ("weights_size", C.c_size_t), ("header", C.c_void_p),
                ("kv_buffer", C.c_void_p), ("kv_size", C.c_size_t),
                ("scratch_buffer", C.c_void_p), ("scratch_size", C.c_size_t),
                ("scratch_head", C.c_size_t), ("scratch_base_offset", C.c_size_t)]


def ref_matmul(A, B):
    """Reference q_matmul_f32_avx2 on dense row-major A[M,K], B[K,N]."""
    R = ref()
    A, B = aligned_copy(f32(A)), aligned_copy(f32(B))
    M, K = A.shape
    _, N = B.shape
    Cm = aligned_empty((M, N), np.float32)
    ctx = _RefCtx()
    assert R.q_alloc_arena(C.addressof(ctx), K * N * 4 + 4096) == Q_OK
    ta, k1 = make_tensor(A.ctypes.data, (M, K, 1, 1), (K * 4, 4, 4, 4), Q_F32)
    tb, k2 = make_tensor(B.ctypes.data, (K, N, 1, 1), (N * 4, 4, 4, 4), Q_F32)
    tc, k3 = make_tensor(Cm.ctypes.data, (M, N, 1, 1), (N * 4, 4, 4, 4), Q_F32)
    rc = R.q_matmul_f32_avx2(C.addressof(ta), C.addressof(tb), C.addressof(tc), C.addressof(ctx))
    R.q_free_memory(C.addressof(ctx))
    return rc, Cm.copy()


def ref_causal_mask(m: np.ndarray, v: float, ne=None, dtype=Q_F32, offset: int = 0):
    """Reference q_causal_mask_f32_avx2 on a copy of m [rows][ld] (32-byte
    aligned plus `offset` bytes); ne defaults to (rows, rows).  Returns
    (rc, matrix)."""
    R = ref()
    rows, ld = m.shape
    raw = aligned_empty((rows * ld + 16,), np.float32, 64)
    o = raw[offset // 4: offset // 4 + rows * ld].reshape(rows, ld)
    o[...] = m
    ne = ne or (rows, rows)
    t, k = make_tensor(o.ctypes.data, (ne[0], ne[1], 1, 1), (ld * 4, 4, 4, 4), dtype)
    rc = R.q_causal_mask_f32_avx2(C.addressof(t), C.c_float(v))
    return rc, o.copy()


class _RefModel(C.Structure):
    """q_llama_model of reference include/qorus_types.h:265-286 (x86-64)."""
    _fields_ = [("config", C.c_uint32 * 9), ("token_embd", C.c_void_p), ("output_norm", C.c_void_p),
                ("output", C.c_void_p), ("layers", C.c_void_p), ("rope_freqs", C.c_void_p),
                ("rope_cache_enabled", C.c_bool), ("rope_cos_cache", C.c_void_p),
                ("rope_sin_cache", C.c_void_p), ("ctx", C.c_void_p)]


def ref_rope_cache(tmp_dir, head_dim: int, max_seq: int, base: float):
    """The RoPE cos/sin cache [max_seq][head_dim] that the reference's own
    llama_build_graph builds (src/models/model.c:625-665), from a file in the
    reference's layout (model.c:352-618: FP32 output, [in, out] shapes) whose
    tensors are zero.  Returns (rc, cos, sin)."""
    R = ref()
    R.q_init_memory.restype = C.c_int
    R.q_init_memory.argtypes = [C.c_void_p, C.c_char_p]
    R.q_alloc_arena.restype = C.c_int
    R.q_alloc_arena.argtypes = [C.c_void_p, C.c_size_t]
    R.llama_build_graph.restype = C.c_int
    R.llama_build_graph.argtypes = [C.c_void_p, C.c_void_p]
    R.q_free_memory.restype = None
    R.q_free_memory.argtypes = [C.c_void_p]
    vocab, n_heads, n_layers = 64, 2, 1
    dim = head_dim * n_heads
    hidden, kvd = dim, dim
    q4 = lambda rows, cols: rows * (cols // 32) * 20
    size = 64 + _al(vocab * dim * 4) * 2 + _al(dim * 4)
    size += n_layers * (2 * _al(dim * 4) + 2 * _al(q4(dim, dim)) + 2 * _al(q4(dim, kvd)) + 3 * _al(q4(dim, hidden)))
    head = struct.pack("<9I2f5I", 0x514F5231, 3, vocab, dim, hidden, n_layers, n_heads, n_heads, max_seq,
                       base, 1e-5, 0, 0, 0, 0, 0)
    path = Path(tmp_dir) / "ref_rope_layout.qorus"
    path.write_bytes(head + bytes(size - 64))
    ctx = _RefCtx()
    model = _RefModel()
    rc = R.q_init_memory(C.addressof(ctx), str(path).encode())
    cos = sin = None
    if rc == Q_OK:
        rc = R.q_alloc_arena(C.addressof(ctx), 2 * max_seq * head_dim * 4 + (1 << 20))
    if rc == Q_OK:
        rc = R.llama_build_graph(C.addressof(ctx), C.addressof(model))
    if rc == Q_OK and model.rope_cache_enabled:
        n = max_seq * head_dim
        cos = np.ctypeslib.as_array((C.c_float * n).from_address(model.rope_cos_cache)).reshape(max_seq, head_dim).copy()
        sin = np.ctypeslib.as_array((C.c_float * n).from_address(model.rope_sin_cache)).reshape(max_seq, head_dim).copy()
    R.q_free_memory(C.addressof(ctx))
    return rc, cos, sin


# ---------------------------------------------------------------------------
# .qorus v3 layout (corrected Llama-3 shapes, Q4_0 LM head) -- an independent
# restatement of the tensor order of reference src/models/model.c:352-618.
# ---------------------------------------------------------------------------

HEADER_FMT = "<11I5I"  # magic..max_seq_len as u32 (floats re-read below)


def parse_header(blob: bytes | np.ndarray) -> dict:
    b = bytes(blob[:64])
    (magic, version, vocab, dim, hidden, n_layers, n_heads, n_kv, max_seq) = struct.unpack_from("<9I", b, 0)
    rope_base, eps = struct.unpack_from("<2f", b, 36)
    return dict(magic=magic, version=version, vocab=vocab, dim=dim, hidden=hidden,
                n_layers=n_layers, n_heads=n_heads, n_kv=n_kv, max_seq=max_seq,
                rope_base=rope_base, eps=eps)


def _al(n: int) -> int:
    return (n + 63) & ~63


def model_layout(h: dict) -> dict:
    """Byte offsets of every tensor of a v3 file."""
    dim, hid, vocab = h["dim"], h["hidden"], h["vocab"]
    hd = dim // h["n_heads"]
    kvd = h["n_kv"] * hd
    q4 = lambda rows, cols: rows * (cols // 32) * 20
    off = 64
    lay = {}

    def put(name, nbytes):
        nonlocal off
        lay[name] = off
        off += _al(nbytes)

    put("token_embd", vocab * dim * 4)
    put("output_norm", dim * 4)
    put("output", q4(vocab, dim))
    for l in range(h["n_layers"]):
        put(f"{l}.attn_norm", dim * 4)
        put(f"{l}.wq", q4(dim, dim))
        put(f"{l}.wk", q4(kvd, dim))
        put(f"{l}.wv", q4(kvd, dim))
        put(f"{l}.wo", q4(dim, dim))
        put(f"{l}.ffn_norm", dim * 4)
        put(f"{l}.w_gate", q4(hid, dim))
        put(f"{l}.w_up", q4(hid, dim))
        put(f"{l}.w_down", q4(dim, hid))
    lay["_size"] = off
    return lay


class _OrModel(C.Structure):
    _fields_ = [("vocab", C.c_uint32), ("dim", C.c_uint32), ("hidden", C.c_uint32),
                ("n_layers", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("max_seq", C.c_uint32), ("rope_base", C.c_float), ("eps", C.c_float),
                ("embd", C.c_void_p), ("output_norm", C.c_void_p), ("lm_head", C.c_void_p),
                ("attn_norm", C.c_void_p), ("wq", C.c_void_p), ("wk", C.c_void_p),
                ("wv", C.c_void_p), ("wo", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("w_gate", C.c_void_p), ("w_up", C.c_void_p), ("w_down", C.c_void_p),
                ("kv", C.c_void_p)]


class DecodeOracle:
    """or_decode_step over a v3 model blob (numpy uint8) and a host KV cache
    [L][n_kv][max_seq][2][head_dim] float32 that the step updates in place."""

    def __init__(self, blob: np.ndarray, kv: np.ndarray):
        self.blob = blob
        self.kv = kv
        h = parse_header(blob)
        self.h = h
        lay = model_layout(h)
        base = blob.ctypes.data
        L = h["n_layers"]
        arr = lambda key: (C.c_void_p * L)(*[base + lay[f"{l}.{key}"] for l in range(L)])
        self._arrays = {k: arr(k) for k in ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm",
                                            "w_gate", "w_up", "w_down")}
        m = _OrModel()
        m.vocab, m.dim, m.hidden = h["vocab"], h["dim"], h["hidden"]
        m.n_layers, m.n_heads, m.n_kv_heads = L, h["n_heads"], h["n_kv"]
        m.max_seq, m.rope_base, m.eps = h["max_seq"], h["rope_base"], h["eps"]
        m.embd = base + lay["token_embd"]
        m.output_norm = base + lay["output_norm"]
        m.lm_head = base + lay["output"]
        for k, a in self._arrays.items():
            setattr(m, k, C.cast(a, C.c_void_p))
        m.kv = kv.ctypes.data
        self.m = m

    def step(self, token: int, pos: int):
        logits = np.empty(self.h["vocab"], dtype=np.float32)
        tok = lib().or_decode_step(C.addressof(self.m), token, pos, logits.ctypes.data)
        return int(tok), logits

    def fill(self, token: int, pos: int):
        """The step's cache rows only (no LM head)."""
        lib().or_decode_step(C.addressof(self.m), token, pos, None)


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def available_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
