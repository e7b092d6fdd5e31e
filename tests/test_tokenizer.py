"""The BPE tokenizer (q_tokenizer_load / encode / decode / free; host code in
libqorus_hip.so, no GPU needed) against the oracle's restatement
(oracle/tokenizer.py) and, where oracle/_ref is built, the reference's own
bpe.c: the same codes and the same ids/text on random and adversarial
tokenizers, every load error, and the reference's own tokenizer test
programs compiled against include/qorus.h (ending as they do against the
reference library).

Bars: bit-exact (token ids, bytes, return codes).
"""
import ctypes as C
import os
import random
import subprocess
from pathlib import Path

import numpy as np
import pytest

import qorus_amd as qa
from oracle import oracle as orc
from oracle import tokenizer as otk

REPO = Path(__file__).resolve().parent.parent
needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built (needs /root/reference)")


def bind(L):
    L.q_tokenizer_load.argtypes = [C.c_void_p, C.c_char_p]
    L.q_tokenizer_load.restype = C.c_int
    L.q_tokenizer_encode.argtypes = [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_bool,
                                     C.c_bool]
    L.q_tokenizer_encode.restype = C.c_int
    L.q_tokenizer_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_size_t]
    L.q_tokenizer_decode.restype = C.c_int
    L.q_tokenizer_free.argtypes = [C.c_void_p]
    L.q_tokenizer_free.restype = None
    return L


class Lib:
    """One library's tokenizer calls on a q_tokenizer it owns."""

    def __init__(self, L):
        self.L = bind(L)
        self.t = qa.QTokenizer()

    def load(self, path):
        return self.L.q_tokenizer_load(C.byref(self.t), str(path).encode())

    def encode(self, text, max_tokens, bos=False, eos=False):
        out = (C.c_uint32 * max(max_tokens, 1))()
        n = C.c_uint32(0xDEADBEEF)
        rc = self.L.q_tokenizer_encode(C.byref(self.t), text, out, C.byref(n), max_tokens, bos, eos)
        return rc, (list(out[:n.value]) if rc == 0 else [])

    def decode(self, ids, size):
        arr = (C.c_uint32 * max(len(ids), 1))(*ids)
        buf = C.create_string_buffer(max(size, 1))
        rc = self.L.q_tokenizer_decode(C.byref(self.t), arr, len(ids), buf, size)
        return rc, (buf.value if size > 0 else b"")

    def free(self):
        self.L.q_tokenizer_free(C.byref(self.t))


def libs():
    out = [("hip", Lib(qa.lib()))]
    if orc.ref_available():
        out.append(("ref", Lib(orc.ref())))
    return out


def random_tokenizer(rng, vocab_size, n_merges, hi_ids=False):
    vocab = [bytes(rng.integers(1, 256, rng.integers(1, 6)).astype(np.uint8)) for _ in range(vocab_size)]
    for i in range(min(256, vocab_size)):
        vocab[i] = bytes([i])  # id 0 is a NUL byte: it decodes to nothing (strlen)
    lo = 256 if vocab_size > 256 else 0
    merges = []
    for _ in range(n_merges):
        a = int(rng.integers(0, min(vocab_size, 300)))
        b = int(rng.integers(0, min(vocab_size, 300)))
        m = int(rng.integers(lo, vocab_size))
        merges.append((a, b, m))
    if hi_ids:
        # rules whose table keys collide: (x, 65536 + y) and (x + 1, y) share
        # (x << 16) | (65536 + y) == ((x + 1) << 16) | y
        for x, y in [(1, 2), (108, 108), (32, 101), (7, 7)]:
            merges.append((x, 65536 + y, int(rng.integers(lo, vocab_size))))
            merges.append((x + 1, y, int(rng.integers(lo, vocab_size))))
            merges.append((x, y, 65536 + y))
    bos, eos, pad = vocab_size - 3, vocab_size - 2, vocab_size - 1
    return vocab, merges, bos, eos, pad


def random_texts(rng, n):
    out = [b"hello world", b"aaaaaaa", b"\x01\x02\x01\x02\x01", b"llll", b" " * 9]
    for _ in range(n):
        k = int(rng.integers(1, 60))
        alphabet = rng.choice([4, 8, 40, 255])
        out.append(bytes((rng.integers(1, alphabet + 1, k)).astype(np.uint8)))
    return out


@pytest.mark.parametrize("vocab_size,n_merges,hi", [(300, 40, False), (200, 25, False), (70000, 60, True),
                                                    (259, 0, False)])
def test_encode_decode_against_oracle_and_reference(tmp_path, vocab_size, n_merges, hi):
    rng = np.random.default_rng(vocab_size + n_merges)
    vocab, merges, bos, eos, pad = random_tokenizer(rng, vocab_size, n_merges, hi)
    path = tmp_path / "tok.bin"
    otk.write(path, vocab, merges, bos, eos, pad)
    rc, ot = otk.load(path)
    assert rc == 0
    impl = libs()
    for _, L in impl:
        assert L.load(path) == 0
        assert L.t.initialized and L.t.vocab_size == vocab_size and L.t.num_merges == len(merges)
    for text in random_texts(rng, 40):
        for mt, bos_, eos_ in [(len(text) + 2, False, False), (len(text) + 2, True, True), (3, False, True)]:
            want = otk.encode(ot, text, mt, bos_, eos_)
            for name, L in impl:
                got = L.encode(text, mt, bos_, eos_)
                assert got == want, (name, text, mt, bos_, eos_, got, want)
        rc, ids = otk.encode(ot, text, len(text) + 2, True, True)
        ids = ids + [vocab_size + 5]  # out of range: skipped
        for size in (1, 2, 5, 64, 4096):
            want = otk.decode(ot, ids, size)
            for name, L in impl:
                assert L.decode(ids, size) == want, (name, text, size)
    for _, L in impl:
        L.free()
        assert not L.t.initialized and not L.t.vocab


def test_table_key_collisions_change_the_merge(tmp_path):
    """A loaded tokenizer looks rules up by the key (id1 << 16) | id2, the
    last rule of a key answering.  (2, 65538) and (3, 2) share the key
    0x30002: on "\x02\x02\x03" rule (2, 3) makes [2, 65538], then rule
    (2, 65538) merges with rule (3, 2)'s id 301 -- while the same rules
    assembled by hand (no table) give 300."""
    vocab = [bytes([i]) for i in range(256)] + [b"w%d" % i for i in range(65600 - 256)]
    vs = len(vocab)
    merges = [(2, 65538, 300), (3, 2, 301), (2, 3, 65538)]
    path = tmp_path / "coll.bin"
    otk.write(path, vocab, merges, vs - 3, vs - 2, vs - 1)
    rc, ot = otk.load(path)
    assert rc == 0
    assert otk.encode(ot, b"\x02\x02\x03", 8, False, False) == (0, [301])
    hand = otk.Tok(ot.vocab, merges, vs - 3, vs - 2, vs - 1, table=False)
    assert otk.encode(hand, b"\x02\x02\x03", 8, False, False) == (0, [300])
    for name, L in libs():
        assert L.load(path) == 0
        assert L.encode(b"\x02\x02\x03", 8) == (0, [301]), name
        L.free()


def test_hand_built_tokenizer_uses_rule_ids():
    """The reference tests assemble q_tokenizer by hand (no table; merged ids
    may lie outside the vocabulary): the rule's own merged id is used."""
    for name, L in libs():
        t = L.t
        t.vocab_size = 256
        t.num_merges = 2
        merges = (C.c_uint32 * 6)(108, 108, 500, 104, 101, 501)
        t.merges = C.cast(merges, C.c_void_p)
        t.vocab = None
        t.merge_hash_table = None
        t.bos_token_id, t.eos_token_id, t.pad_token_id = 256, 257, 258
        t.initialized = True
        assert L.encode(b"hello", 16) == (0, [501, 500, 111]), name
        assert L.encode(b"hello", 16, True, True) == (0, [256, 501, 500, 111, 257]), name
        assert L.encode(b"hello", 2) == (-8, []), name
        t.merges = None
        t.num_merges = 0
        t.initialized = False


def test_encode_and_decode_codes():
    for name, L in libs():
        assert L.L.q_tokenizer_encode(None, b"x", None, None, 4, False, False) == -10
        t = L.t
        t.initialized = False
        assert L.encode(b"x", 4) == (-10, []), name
        assert L.decode([1], 4) == (-10, b""), name
        t.vocab_size, t.bos_token_id, t.eos_token_id, t.pad_token_id = 256, 256, 257, 258
        t.initialized = True
        assert L.encode(b"x", 0) == (-15, []), name
        assert L.encode(b"", 1, True, True) == (-8, []), name
        assert L.encode(b"", 2, True, True) == (0, [256, 257]), name
        assert L.encode(b"", 4) == (0, []), name
        assert L.decode([1], 0)[0] == -15, name
        t.initialized = False


def load_error_cases(tmp_path):
    v = [bytes([i]) if i else b"\x01" for i in range(256)] + [b"<s>", b"</s>", b"<pad>"]
    cases = {}

    def mk(name, **kw):
        p = tmp_path / f"{name}.bin"
        args = dict(vocab=v, merges=[(104, 105, 258)], bos=256, eos=257, pad=258)
        args.update(kw)
        otk.write(p, **args)
        cases[name] = p
        return p

    mk("ok")
    mk("magic", magic=0x12345678)
    mk("version", version=2)
    mk("vocab0", vocab_size=0)
    mk("vocabbig", vocab_size=1000001)
    mk("mergesbig", n_merges=1000001)
    mk("mergeid", merges=[(104, 259, 258)])
    mk("mergedid", merges=[(104, 105, 259)])
    p = mk("trunc_vocab")
    data = p.read_bytes()
    p.write_bytes(data[:32 + 100])
    p = mk("trunc_merge")
    data = p.read_bytes()
    p.write_bytes(data[:-5])
    p = mk("trunc_header")
    p.write_bytes(p.read_bytes()[:20])
    p = mk("empty_entry")
    data = bytearray(p.read_bytes())
    data[32] = 0  # first entry's length
    p.write_bytes(bytes(data))
    cases["missing"] = tmp_path / "does_not_exist.bin"
    return cases


def test_load_errors(tmp_path):
    cases = load_error_cases(tmp_path)
    expect = {"ok": 0, "magic": -6, "version": -10, "vocab0": -15, "vocabbig": -15, "mergesbig": -15,
              "mergeid": -10, "mergedid": -10, "trunc_vocab": -2, "trunc_merge": -2, "trunc_header": -2,
              "empty_entry": -15, "missing": -2}
    for name, path in cases.items():
        assert otk.load(path)[0] == expect[name], name
        for lname, L in libs():
            rc = L.load(path)
            assert rc == expect[name], (lname, name, rc)
            if rc == 0:
                L.free()
    for _, L in libs():
        assert L.L.q_tokenizer_load(None, b"x") == -10
        assert L.L.q_tokenizer_load(C.byref(L.t), None) == -10


def test_load_fuzz_matches_oracle(tmp_path):
    """Seeded corruptions of a valid tokenizer file (truncations, flipped
    bytes, rewritten header words, zeroed or enlarged entry lengths): this
    library's loader returns the oracle's code for every one and, where both
    accept the file, encodes and decodes as the oracle does.  (Under the
    host-sanitizer build this is also the loader's memory-safety check.)"""
    rng = random.Random(2027)
    v = [bytes([i]) if i else b"\x01" for i in range(256)] + [b"ab", b"<s>", b"</s>", b"<pad>"]
    base = tmp_path / "base.bin"
    otk.write(base, vocab=v, merges=[(97, 98, 256), (256, 256, 258), (104, 105, 259)], bos=257, eos=258, pad=259)
    good = base.read_bytes()
    L = Lib(qa.lib())
    n_ok = 0
    for k in range(300):
        d = bytearray(good)
        kind = k % 5
        if kind == 0:
            d = d[:rng.randrange(0, len(d))]
        elif kind == 1:
            for _ in range(rng.randint(1, 4)):
                d[rng.randrange(len(d))] = rng.randrange(256)
        elif kind == 2:
            w = rng.choice([2, 3, 4, 5, 6, 7])  # vocab, merges, bos, eos, pad, reserved
            d[4 * w:4 * w + 4] = rng.choice([0, 1, 5, 261, 262, 70000, 1000000, 1000001, 0xFFFFFFFF]).to_bytes(4, "little")
        elif kind == 3:
            d[32 + 2 * rng.randrange(200)] = rng.choice([0, 1, 2, 200, 255])
        else:
            i = rng.randrange(len(good) - 12, len(good) - 3)
            d[i:i + 4] = rng.choice([96, 255, 259, 260, 261, 65536]).to_bytes(4, "little")
        path = tmp_path / f"f{k}.bin"
        path.write_bytes(bytes(d))
        want_rc, ot = otk.load(path)
        rc = L.load(path)
        assert rc == want_rc, (k, kind, rc, want_rc)
        if rc == 0:
            n_ok += 1
            for text in (b"abab hi", b"hhii", b"\x05\x06abab"):
                assert L.encode(text, 16, True, True) == otk.encode(ot, text, 16, True, True), (k, text)
            ids = [1, 97, 256, 258, 259, 260, 7]
            assert L.decode(ids, 64) == otk.decode(ot, ids, 64), k
            L.free()
    assert 0 < n_ok < 300


def test_python_front_end(tmp_path):
    path = tmp_path / "bytes.bin"
    qa.write_tokenizer(path, qa.byte_level_vocab(), merges=[(108, 108, 258)])
    tok = qa.Tokenizer(path)
    assert tok.bos == 256 and tok.eos == 257
    ids = tok.encode("hello", add_bos=True)
    assert ids == [256, 104, 101, 258, 111]  # pad id 258 doubles as the 'll' merge here
    assert tok.decode([256, 104, 101, 108, 108, 111, 257]) == b"hello"
    tok.close()


# The reference's own tokenizer test programs, built by `make -C oracle
# callers` against include/qorus.h + libqorus_hip.so and against the
# reference library; both must end the same way.
# (test_tokenizer_adversarial.c does not compile against the reference's own
# headers either and is left out.)
TOK_CALLERS = ["test_bpe_tokenizer", "test_bpe_tokenizer_adversarial", "test_bpe_soft_delete",
               "test_tokenizer_free_complete"]


@pytest.mark.parametrize("name", TOK_CALLERS)
def test_reference_tokenizer_programs(tmp_path, name):
    exe = REPO / "oracle" / "_ref" / "callers" / name
    exe_ref = REPO / "oracle" / "_ref" / "callers_ref" / name
    if not exe.exists() or not exe_ref.exists():
        pytest.skip("reference callers not built (make -C oracle callers needs the reference sources)")

    def run(e):
        # a fresh directory per run (the programs delete their files), with
        # tokenizer.bin in the layout of the reference converter's byte-level
        # tokenizer
        d = tmp_path / e.parent.name
        d.mkdir()
        otk.write(d / "tokenizer.bin", qa.byte_level_vocab(), [], 256, 257, 258)
        p = subprocess.run([str(e)], cwd=d, capture_output=True, text=True, timeout=300)
        return p.returncode, (p.stdout + p.stderr)[-2000:]

    rc, out = run(exe)
    rc_ref, out_ref = run(exe_ref)
    print(f"{name}: hip rc={rc} | reference rc={rc_ref}")
    assert rc == rc_ref, f"{name}: exit {rc}, reference library {rc_ref}\n{out}\n--- reference ---\n{out_ref}"
