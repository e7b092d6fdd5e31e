"""CPU restatement of the reference's byte-level BPE tokenizer (test
infrastructure only: the parity checker of q_tokenizer_* in libqorus_hip.so,
never part of the product path).

Follows reference src/tokenizer/bpe.c:
  load      bpe.c:263-... (header, vocab, merges, validation order and codes)
  table     bpe.c:105-219 (merge lookup by key (id1 << 16) | id2 in a chained
            hash table with head insertion: a key answers with the LAST rule of
            that key in file order)
  encode    bpe.c:568-808 (bytes -> ids, greedy merge passes, BOS/EOS, codes)
  decode    bpe.c:811-866 (special/out-of-range ids skipped, the buffer bound)

Pinned (tests/test_tokenizer.py) against oracle/_ref (the reference's bpe.c
compiled from its sources) on random and adversarial tokenizers, including
vocabularies past 65536 ids where different rules share a table key, every
load error, and the decode bound.
"""
from __future__ import annotations

import struct

Q_OK = 0
Q_ERR_FILE_OPEN = -2
Q_ERR_INVALID_MAGIC = -6
Q_ERR_ARENA_OOM = -8
Q_ERR_INVALID_ARG = -10
Q_ERR_INVALID_SIZE = -15

MAGIC = 0x51544B52
VERSION = 1
MAX_TEXT = 1024 * 1024
DEAD = 0xFFFFFFFF


class Tok:
    def __init__(self, vocab, merges, bos, eos, pad, table=True):
        self.vocab = vocab            # list of bytes (or None for hand-made entries)
        self.merges = merges          # list of (id1, id2, merged)
        self.bos, self.eos, self.pad = bos, eos, pad
        self.table = table            # built by load (bpe.c:105-156)

    def merged_of(self, i):
        """bpe.c:531-545: the table's answer for rule i's key, else the rule's own."""
        if not self.table:
            return self.merges[i][2]
        a, b, _ = self.merges[i]
        key = (a << 16) | b
        for j in range(len(self.merges) - 1, -1, -1):   # head insertion: last rule first
            x, y, m = self.merges[j]
            if ((x << 16) | y) == key:
                return m
        return self.merges[i][2]


def load(path):
    """-> (rc, Tok or None)"""
    try:
        f = open(path, "rb")
    except OSError:
        return Q_ERR_FILE_OPEN, None
    with f:
        data = f.read()
    off = 0

    def u32():
        nonlocal off
        if off + 4 > len(data):
            raise EOFError
        v = struct.unpack_from("<I", data, off)[0]
        off += 4
        return v

    try:
        if u32() != MAGIC:
            return Q_ERR_INVALID_MAGIC, None
        if u32() != VERSION:
            return Q_ERR_INVALID_ARG, None
        vocab_size, n_merges, bos, eos, pad, _ = (u32() for _ in range(6))
        if vocab_size == 0 or vocab_size > 1000000:
            return Q_ERR_INVALID_SIZE, None
        if n_merges > 1000000:
            return Q_ERR_INVALID_SIZE, None
        vocab = []
        for _ in range(vocab_size):
            if off + 1 > len(data):
                raise EOFError
            n = data[off]
            off += 1
            if n == 0:
                return Q_ERR_INVALID_SIZE, None
            if off + n > len(data):
                raise EOFError
            vocab.append(data[off:off + n])
            off += n
        merges = []
        for _ in range(n_merges):
            a, b, m = u32(), u32(), u32()
            if a >= vocab_size or b >= vocab_size or m >= vocab_size:
                return Q_ERR_INVALID_ARG, None
            merges.append((a, b, m))
    except EOFError:
        return Q_ERR_FILE_OPEN, None
    return Q_OK, Tok(vocab, merges, bos, eos, pad, table=n_merges > 0)


def apply_merges(tok, ids):
    """bpe.c:568-654: passes over the rules in order until nothing changes;
    each rule scans the live tokens left to right, merging (id1, id2) into
    the first slot and killing the second; the scan resumes after it."""
    if not tok.merges or len(ids) < 2:
        return ids
    ids = list(ids)
    merged = [tok.merged_of(i) for i in range(len(tok.merges))]
    changed = True
    while changed:
        changed = False
        for r, (a, b, _) in enumerate(tok.merges):
            n = len(ids)
            j = 0
            while j < n:
                if ids[j] == DEAD:
                    j += 1
                    continue
                k = j + 1
                while k < n and ids[k] == DEAD:
                    k += 1
                if k >= n:
                    break
                if ids[j] == a and ids[k] == b:
                    ids[j] = merged[r]
                    ids[k] = DEAD
                    changed = True
                j += 1
        ids = [t for t in ids if t != DEAD]
    return ids


def encode(tok, text: bytes, max_tokens: int, add_bos: bool, add_eos: bool):
    """-> (rc, ids).  text is the C string's bytes (no NUL)."""
    if max_tokens == 0:
        return Q_ERR_INVALID_SIZE, []
    if len(text) == 0:
        need = int(add_bos) + int(add_eos)
        if need > max_tokens:
            return Q_ERR_ARENA_OOM, []
        return Q_OK, ([tok.bos] if add_bos else []) + ([tok.eos] if add_eos else [])
    if len(text) > MAX_TEXT:
        return Q_ERR_ARENA_OOM, []
    ids = [c if c < len(tok.vocab) else tok.pad for c in text]
    ids = apply_merges(tok, ids)
    out = ([tok.bos] if add_bos else []) + ids + ([tok.eos] if add_eos else [])
    if len(out) > max_tokens:
        return Q_ERR_ARENA_OOM, []
    return Q_OK, out


def decode(tok, ids, buf_size: int):
    """-> (rc, bytes written before the NUL)."""
    if buf_size == 0:
        return Q_ERR_INVALID_SIZE, b""
    out = b""
    for t in ids:
        if t in (tok.bos, tok.eos, tok.pad) or t >= len(tok.vocab) or tok.vocab[t] is None:
            continue
        s = tok.vocab[t].split(b"\0", 1)[0]
        if len(out) + len(s) >= buf_size - 1:
            return Q_ERR_ARENA_OOM, out
        out += s
    return Q_OK, out


def write(path, vocab, merges, bos, eos, pad, magic=MAGIC, version=VERSION, vocab_size=None, n_merges=None):
    """A tokenizer file in the reference's layout (with optional wrong header
    fields, for the load-error tests)."""
    with open(path, "wb") as f:
        f.write(struct.pack("<8I", magic, version, len(vocab) if vocab_size is None else vocab_size,
                            len(merges) if n_merges is None else n_merges, bos, eos, pad, 0))
        for v in vocab:
            f.write(bytes([len(v)]) + v)
        for a, b, m in merges:
            f.write(struct.pack("<3I", a, b, m))
