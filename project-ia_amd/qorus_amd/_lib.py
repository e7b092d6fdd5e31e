"""ctypes bindings of libqorus_hip.so."""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent  # project-ia_amd/
# QORUS_HIP_LIB selects another build of the same library (the host-sanitizer
# build of `make -C project-ia_amd asan`, for the CPU tests of the host code).
LIB_PATH = Path(os.environ.get("QORUS_HIP_LIB") or PKG_DIR / "build" / "libqorus_hip.so")

Q_OK = 0
Q_F32 = 0
Q_Q8_0 = 1
Q_Q4_0 = 2

ERR = {
    0: "Q_OK", -1: "Q_ERR_NULL_PTR", -2: "Q_ERR_FILE_OPEN", -3: "Q_ERR_FILE_STAT",
    -4: "Q_ERR_FILE_TOO_SMALL", -5: "Q_ERR_MMAP_FAILED", -6: "Q_ERR_INVALID_MAGIC",
    -7: "Q_ERR_ALLOC_FAILED", -8: "Q_ERR_ARENA_OOM", -9: "Q_ERR_INVALID_CONFIG",
    -10: "Q_ERR_INVALID_ARG", -11: "Q_ERR_ALIASING", -12: "Q_ERR_OVERFLOW",
    -13: "Q_ERR_MISALIGNED", -14: "Q_ERR_INVALID_DTYPE", -15: "Q_ERR_INVALID_SIZE",
}
globals().update({v: k for k, v in ERR.items()})


class QorusError(RuntimeError):
    pass


class QTensor(C.Structure):
    """q_tensor: 128 bytes, aligned(64) in C (reference qorus_types.h:205-213)."""
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


class _AlignedTensor:
    """A QTensor placed in 64-byte aligned host memory (the C type is
    aligned(64), so compilers may assume that alignment)."""

    def __init__(self, ptr: int, ne, nb, dtype: int, name: bytes = b""):
        raw = np.zeros(128 + 64, dtype=np.uint8)
        off = (-raw.ctypes.data) % 64
        self._raw = raw
        self.t = QTensor.from_buffer(raw, off)
        self.t.data = ptr
        for i in range(4):
            self.t.ne[i] = ne[i]
            self.t.nb[i] = nb[i]
        self.t.type = dtype
        self.t.name = name[:31]

    @property
    def ref(self):
        return C.byref(self.t)

    @property
    def addr(self) -> int:
        return C.addressof(self.t)


def q4_tensor(ptr: int, M: int, N: int, nb0: int | None = None) -> _AlignedTensor:
    """Q4_0 [M rows, N cols] view (strides of reference model.c:258-273)."""
    rb = (N // 32) * 20 if nb0 is None else nb0
    return _AlignedTensor(ptr, (M, N, 1, 1), (rb, 20, 20, 20), Q_Q4_0)


def f32_tensor(ptr: int, n: int) -> _AlignedTensor:
    """Contiguous 1-D fp32 view (nb[0] = n*4, as reference add/mul expect)."""
    return _AlignedTensor(ptr, (n, 1, 1, 1), (n * 4, 4, 4, 4), Q_F32)


_lib = None
vp = C.c_void_p
u32 = C.c_uint32
u64 = C.c_uint64
f32 = C.c_float
i32 = C.c_int


def _sig(L, name, res, *args):
    fn = getattr(L, name)
    fn.restype = res
    fn.argtypes = list(args)


def lib():
    """Load libqorus_hip.so (raises QorusError if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise QorusError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C project-ia_amd)")
    L = C.CDLL(str(LIB_PATH))
    # runtime
    _sig(L, "qh_available", i32)
    _sig(L, "qh_last_error", C.c_char_p)
    _sig(L, "qh_arch_name", C.c_char_p)
    _sig(L, "qh_malloc", i32, C.POINTER(vp), C.c_size_t)
    _sig(L, "qh_free", i32, vp)
    _sig(L, "qh_memcpy_htod", i32, vp, vp, C.c_size_t)
    _sig(L, "qh_memcpy_dtoh", i32, vp, vp, C.c_size_t)
    _sig(L, "qh_memcpy_dtod", i32, vp, vp, C.c_size_t, vp)
    _sig(L, "qh_memset", i32, vp, i32, C.c_size_t, vp)
    _sig(L, "qh_stream_create", i32, C.POINTER(vp))
    _sig(L, "qh_stream_destroy", i32, vp)
    _sig(L, "qh_stream_synchronize", i32, vp)
    _sig(L, "qh_device_synchronize", i32)
    _sig(L, "qh_event_create", i32, C.POINTER(vp))
    _sig(L, "qh_event_destroy", i32, vp)
    _sig(L, "qh_event_record", i32, vp, vp)
    _sig(L, "qh_event_synchronize", i32, vp)
    _sig(L, "qh_event_elapsed_ms", i32, vp, vp, C.POINTER(f32))
    _sig(L, "qh_stream_begin_capture", i32, vp)
    _sig(L, "qh_stream_end_capture", i32, vp, C.POINTER(vp))
    _sig(L, "qh_graph_launch", i32, vp, vp)
    _sig(L, "qh_graph_destroy", i32, vp)
    # memory tiers
    _sig(L, "q_init_memory", i32, vp, C.c_char_p)
    _sig(L, "q_init_memory_ex", i32, vp, C.c_char_p, i32)
    _sig(L, "q_alloc_kv_cache", i32, vp, C.c_size_t)
    _sig(L, "q_alloc_arena", i32, vp, C.c_size_t)
    _sig(L, "q_arena_alloc", vp, vp, C.c_size_t)
    _sig(L, "q_arena_reset", None, vp)
    _sig(L, "q_free_memory", None, vp)
    _sig(L, "q_strerror", C.c_char_p, i32)
    # q4
    _sig(L, "q_dequantize_q4_0_block_avx2_public", None, vp, vp)
    _sig(L, "q_gemv_q4_f32_avx2", i32, vp, vp, vp)
    _sig(L, "qh_dequantize_q4_0", i32, vp, vp, u64, vp)
    _sig(L, "qh_gemv_workspace_bytes", C.c_size_t, u32)
    _sig(L, "qh_gemv_q4_f32", i32, vp, vp, vp, vp, vp)
    _sig(L, "qh_gemv_q4_f32_add", i32, vp, vp, vp, vp, vp, vp)
    _sig(L, "qh_gemv_prepare", i32, vp, u32, vp, vp)
    _sig(L, "qh_gemv_q4_f32_prepared", i32, vp, vp, vp, u32, vp, vp)
    _sig(L, "qh_gemv_q4_f32_multi", i32, vp, vp, vp, u32, vp, vp, vp)
    _sig(L, "qh_gemm_workspace_bytes", C.c_size_t, u32, u32, u32)
    _sig(L, "qh_gemm_q4_f32", i32, vp, vp, u32, vp, vp, vp)
    _sig(L, "qh_gemm_q4_f32_multi", i32, vp, vp, u32, vp, u32, vp, vp)
    # vector ops
    _sig(L, "q_rmsnorm_f32_avx2", i32, vp, vp, vp, u32, f32)
    _sig(L, "q_rope_f32_avx2", i32, vp, vp, vp, vp, u32)
    _sig(L, "q_silu_f32_avx2", i32, vp, vp, u32)
    _sig(L, "q_softmax_f32_avx2", i32, vp, vp, u32)
    _sig(L, "q_add_f32_avx2", i32, vp, vp, vp)
    _sig(L, "q_matmul_f32_avx2", i32, vp, vp, vp, vp)
    _sig(L, "q_mul_f32_avx2", i32, vp, vp, vp)
    _sig(L, "q_causal_mask_f32_avx2", i32, vp, f32)
    # tokenizer and generation loop (host)
    _sig(L, "q_tokenizer_load", i32, vp, C.c_char_p)
    _sig(L, "q_tokenizer_encode", i32, vp, C.c_char_p, vp, vp, u32, C.c_bool, C.c_bool)
    _sig(L, "q_tokenizer_decode", i32, vp, vp, u32, vp, C.c_size_t)
    _sig(L, "q_tokenizer_free", None, vp)
    _sig(L, "q_generate", i32, vp)
    _sig(L, "qh_causal_mask_f32", i32, vp, u32, u32, f32, vp)
    _sig(L, "qh_rmsnorm_f32", i32, vp, vp, vp, u32, f32, vp)
    _sig(L, "qh_rope_f32", i32, vp, vp, vp, vp, u32, u32, vp)
    _sig(L, "qh_silu_f32", i32, vp, vp, u32, vp)
    _sig(L, "qh_silu_mul_f32", i32, vp, vp, vp, u32, vp)
    _sig(L, "qh_softmax_f32", i32, vp, vp, u32, vp)
    _sig(L, "qh_softmax_workspace_bytes", C.c_size_t, u32)
    _sig(L, "qh_softmax_f32_ws", i32, vp, vp, u32, vp, vp)
    _sig(L, "qh_argmax_workspace_bytes", C.c_size_t, u32)
    _sig(L, "qh_argmax_f32_ws", i32, vp, u32, vp, vp, vp)
    _sig(L, "qh_softmax_argmax_f32_ws", i32, vp, vp, u32, vp, vp, vp)
    _sig(L, "qh_gemv_softmax_workspace_bytes", C.c_size_t, u32)
    _sig(L, "qh_gemv_q4_f32_softmax_argmax", i32, vp, vp, vp, vp, vp, vp, vp)
    _sig(L, "qh_gemv_q4_f32_softmax_argmax_noalloc", i32, vp, vp, vp, vp, vp, vp)
    _sig(L, "qh_add_f32", i32, vp, vp, vp, u32, vp)
    _sig(L, "qh_mul_f32", i32, vp, vp, vp, u32, vp)
    _sig(L, "qh_argmax_f32", i32, vp, u32, vp, vp)
    _optional_sigs(L)
    _lib = L
    return L


def _optional_sigs(L):
    """Entry points added as the build grows; bound when present."""
    opt = [
        ("q_matmul_f32_avx2", i32, vp, vp, vp, vp),
        ("llama_build_graph", i32, vp, vp),
        ("llama_free_graph", None, vp),
        ("llama_forward", i32, vp, vp, vp, u32, u32, vp),
        ("q_sample_token", i32, vp, u32, f32, u32, f32, vp, vp),
        ("qh_llama_generate", i32, vp, vp, u32, u32, u32, vp, vp),
        ("qh_llama_generate_sampled", i32, vp, vp, u32, u32, u32, f32, u32, f32, vp, vp),
        ("qh_sample_set_state", None, u64),
        ("qh_sample_get_state", u64),
    ]
    for name, res, *args in opt:
        if hasattr(L, name):
            _sig(L, name, res, *args)


def check(rc: int, what: str = ""):
    if rc != Q_OK:
        msg = ERR.get(rc, str(rc))
        extra = ""
        try:
            extra = lib().qh_last_error().decode()
        except Exception:
            pass
        raise QorusError(f"{what}: {msg} {extra}".strip())


def gpu_available() -> bool:
    try:
        return bool(lib().qh_available())
    except QorusError:
        return False


class DeviceBuffer:
    """An HBM allocation owned by Python (qh_malloc / qh_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = vp()
        check(lib().qh_malloc(C.byref(p), max(self.nbytes, 1)), "qh_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().qh_memcpy_htod(self.ptr + offset, a.ctypes.data, a.nbytes), "htod")

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().qh_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes), "dtoh")
        return out

    def zero(self, stream=None):
        check(lib().qh_memset(self.ptr, 0, self.nbytes, stream), "memset")

    def free(self):
        if self.ptr:
            lib().qh_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = vp()
        check(lib().qh_stream_create(C.byref(s)), "stream_create")
        self.handle = s.value

    def sync(self):
        check(lib().qh_stream_synchronize(self.handle), "stream_sync")

    def __del__(self):
        try:
            lib().qh_stream_destroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        e = vp()
        check(lib().qh_event_create(C.byref(e)), "event_create")
        self.handle = e.value

    def record(self, stream=None):
        check(lib().qh_event_record(self.handle, stream.handle if isinstance(stream, Stream) else stream),
              "event_record")

    def sync(self):
        check(lib().qh_event_synchronize(self.handle), "event_sync")

    def elapsed_ms(self, end: "Event") -> float:
        ms = f32()
        check(lib().qh_event_elapsed_ms(self.handle, end.handle, C.byref(ms)), "elapsed")
        return float(ms.value)

    def __del__(self):
        try:
            lib().qh_event_destroy(self.handle)
        except Exception:
            pass
