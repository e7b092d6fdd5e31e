"""Python front-end of the library's BPE tokenizer (q_tokenizer_load /
encode / decode / free, host code) and a writer of the tokenizer file it
reads.

File layout (the reference's 'QTKR' v1, src/tokenizer/bpe.c): a 32-byte
little-endian header {magic 0x51544B52, version 1, vocab_size, num_merges,
bos, eos, pad, reserved}, vocab_size entries {u8 length >= 1, bytes}, then
num_merges rules {u32 id1, u32 id2, u32 merged}.
"""
from __future__ import annotations

import ctypes as C
import struct

from ._lib import QorusError, check, lib

TOKENIZER_MAGIC = 0x51544B52
TOKENIZER_VERSION = 1


class QTokenizer(C.Structure):
    """q_tokenizer (include/qorus_types.h), 56 bytes on LP64."""
    _fields_ = [("vocab", C.c_void_p), ("vocab_size", C.c_uint32), ("merges", C.c_void_p),
                ("num_merges", C.c_uint32), ("merge_hash_table", C.c_void_p), ("bos_token_id", C.c_uint32),
                ("eos_token_id", C.c_uint32), ("pad_token_id", C.c_uint32), ("initialized", C.c_bool)]


def write_tokenizer(path, vocab, merges=(), bos=None, eos=None, pad=None):
    """Write vocab (a list of non-empty byte strings of at most 255 bytes) and
    merge rules (id1, id2, merged) in the library's tokenizer file layout.
    bos/eos/pad default to the last three vocab entries."""
    n = len(vocab)
    bos = n - 3 if bos is None else bos
    eos = n - 2 if eos is None else eos
    pad = n - 1 if pad is None else pad
    with open(path, "wb") as f:
        f.write(struct.pack("<8I", TOKENIZER_MAGIC, TOKENIZER_VERSION, n, len(merges), bos, eos, pad, 0))
        for v in vocab:
            if not 1 <= len(v) <= 255:
                raise ValueError("vocab entries hold 1..255 bytes")
            f.write(bytes([len(v)]) + bytes(v))
        for a, b, m in merges:
            f.write(struct.pack("<3I", a, b, m))


def byte_level_vocab():
    """The 256 single-byte tokens followed by BOS, EOS and pad (ids 256-258),
    the layout of the reference converter's tokenizer."""
    return [bytes([i]) for i in range(256)] + [b"<|begin_of_text|>", b"<|end_of_text|>",
                                              b"<|finetune_right_pad_id|>"]


class Tokenizer:
    """A loaded tokenizer; encode/decode raise QorusError on a failing code."""

    def __init__(self, path):
        self._lib = lib()
        self.t = QTokenizer()
        check(self._lib.q_tokenizer_load(C.byref(self.t), str(path).encode()), "q_tokenizer_load")

    @property
    def bos(self):
        return self.t.bos_token_id

    @property
    def eos(self):
        return self.t.eos_token_id

    def encode(self, text, max_tokens=None, add_bos=False, add_eos=False):
        data = text.encode() if isinstance(text, str) else bytes(text)
        cap = max_tokens if max_tokens is not None else len(data) + 2
        out = (C.c_uint32 * max(cap, 1))()
        n = C.c_uint32(0)
        check(self._lib.q_tokenizer_encode(C.byref(self.t), data, out, C.byref(n), cap, add_bos, add_eos),
              "q_tokenizer_encode")
        return list(out[:n.value])

    def decode(self, ids, buf_size=None):
        ids = list(ids)
        arr = (C.c_uint32 * max(len(ids), 1))(*ids)
        if buf_size is None:
            buf_size = 2 + sum(len(self._entry(i)) for i in ids)
        buf = C.create_string_buffer(buf_size)
        check(self._lib.q_tokenizer_decode(C.byref(self.t), arr, len(ids), buf, buf_size), "q_tokenizer_decode")
        return buf.value

    def _entry(self, i):
        if i >= self.t.vocab_size:
            return b""
        p = C.cast(self.t.vocab, C.POINTER(C.c_char_p))[i]
        return p or b""

    def close(self):
        if self.t.initialized or self.t.vocab:
            self._lib.q_tokenizer_free(C.byref(self.t))

    def __del__(self):
        try:
            self.close()
        except (QorusError, OSError):
            pass
