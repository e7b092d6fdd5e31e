""".qorus model files, version 3 (Llama-3 shapes as the GEMV consumes them).

The container is the reference's: a 64-byte header (reference
include/qorus_types.h:189-203) followed by the tensors in the order of
reference src/models/model.c:352-618, each padded to 64 bytes.  Version 3
differs from what the reference's converter writes (tools/convert_llama.py)
in three documented ways, all needed for a Llama-3-8B decode to be correct:

* every Q4_0 matrix holds real 20-byte blocks (the reference writer stores
  FP32 bytes in Q4_0 slots);
* matrices are stored [out, in] -- ne[0] = output rows -- which is the
  convention q_gemv_q4_f32_avx2 reads (reference matmul.c:210-211), so
  wk/wv are [kv_dim, dim], w_gate/w_up [hidden, dim], w_down [dim, hidden];
* the LM head ("output") is Q4_0 [vocab, dim] instead of FP32.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Callable

import numpy as np

Q_MAGIC = 0x514F5231
VERSION = 3


@dataclass
class QorusHeader:
    vocab: int
    dim: int
    hidden: int
    n_layers: int
    n_heads: int
    n_kv: int
    max_seq: int
    rope_base: float = 500000.0
    eps: float = 1e-5

    def pack(self) -> bytes:
        b = struct.pack("<9I2f5I", Q_MAGIC, VERSION, self.vocab, self.dim, self.hidden, self.n_layers,
                        self.n_heads, self.n_kv, self.max_seq, self.rope_base, self.eps, 0, 0, 0, 0, 0)
        assert len(b) == 64
        return b

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim


def _al(n: int) -> int:
    return (n + 63) & ~63


def q4_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 32) * 20


def tensor_specs(h: QorusHeader):
    """(name, kind, shape, nbytes) in file order; kind is 'f32' or 'q4'."""
    d, hid, v, kvd = h.dim, h.hidden, h.vocab, h.kv_dim
    specs = [("token_embd", "f32", (v, d), v * d * 4),
             ("output_norm", "f32", (d,), d * 4),
             ("output", "q4", (v, d), q4_bytes(v, d))]
    for l in range(h.n_layers):
        specs += [
            (f"{l}.attn_norm", "f32", (d,), d * 4),
            (f"{l}.wq", "q4", (d, d), q4_bytes(d, d)),
            (f"{l}.wk", "q4", (kvd, d), q4_bytes(kvd, d)),
            (f"{l}.wv", "q4", (kvd, d), q4_bytes(kvd, d)),
            (f"{l}.wo", "q4", (d, d), q4_bytes(d, d)),
            (f"{l}.ffn_norm", "f32", (d,), d * 4),
            (f"{l}.w_gate", "q4", (hid, d), q4_bytes(hid, d)),
            (f"{l}.w_up", "q4", (hid, d), q4_bytes(hid, d)),
            (f"{l}.w_down", "q4", (d, hid), q4_bytes(d, hid)),
        ]
    return specs


def model_layout(h: QorusHeader) -> dict:
    off = 64
    lay = {}
    for name, _, _, nbytes in tensor_specs(h):
        lay[name] = off
        off += _al(nbytes)
    lay["_size"] = off
    return lay


def write_qorus_v3(path, h: QorusHeader, get_tensor: Callable[[str, str, tuple], np.ndarray]) -> int:
    """Stream a v3 file; get_tensor(name, kind, shape) returns float32 data for
    'f32' tensors and uint8 [rows, cols/32*20] AoS Q4_0 blocks for 'q4'."""
    with open(path, "wb") as f:
        f.write(h.pack())
        for name, kind, shape, nbytes in tensor_specs(h):
            a = np.ascontiguousarray(get_tensor(name, kind, shape))
            if a.nbytes != nbytes:
                raise ValueError(f"{name}: {a.nbytes} bytes, expected {nbytes}")
            f.write(a.tobytes(order="C"))
            pad = _al(nbytes) - nbytes
            if pad:
                f.write(b"\0" * pad)
        return f.tell()
