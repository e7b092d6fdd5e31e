"""Adversarial GEMV/GEMM inputs: activation outliers that meet zero weights.

An outlier channel whose weight nibble is 8 in every row ((8 - 8) * s = 0)
adds nothing to sum_j |W_ij x_j|, so the outputs' condition is set by the
ordinary elements only.  Any representation of x whose precision follows
the largest element of a group (a shared exponent) loses the ordinary
elements' low bits there, and the error statistic exposes it.  The
reference's fp32 FMA order is unaffected (a zero product changes no sum).

Cases (kind, count): 'channel' puts one outlier on one channel; 'block' one
outlier in every 32-element block; 'one' / 'all' put `count` equal outliers
(alternating signs) in one block / in every block; 'mixed-one' /
'mixed-all' put four outliers of mag, mag/10, mag/100 and mag/1000.  Every
case draws its columns from one layout, so a single weight matrix (nibble 8
on all of them) serves them all.
"""
from __future__ import annotations

import numpy as np

MAX_PER_BLOCK = 6


def set_nibble8(W: np.ndarray, cols) -> np.ndarray:
    """Copy of the Q4_0 matrix W ([M, N/32*20] bytes) with nibble 8 (weight
    exactly zero) in every row at the given element columns."""
    W = W.copy()
    for j in np.atleast_1d(cols):
        b, e = divmod(int(j), 32)
        byte = 20 * b + (e >> 1)
        if e & 1:
            W[:, byte] = (W[:, byte] & 0x0F) | 0x80
        else:
            W[:, byte] = (W[:, byte] & 0xF0) | 0x08
    return W


class Layout:
    """Outlier columns of an input of width N: a channel, and per block
    MAX_PER_BLOCK distinct element positions (the first `count` are used)."""

    def __init__(self, N: int, rng: np.random.Generator):
        nblk = N // 32
        self.N = N
        self.chan = int(rng.integers(0, N))
        self.one = int(rng.integers(0, nblk))
        self.pos = np.stack([32 * b + rng.permutation(32)[:MAX_PER_BLOCK] for b in range(nblk)])

    def zero_columns(self) -> list:
        return sorted({self.chan} | set(self.pos.reshape(-1).tolist()))

    def columns(self, kind: str, count: int):
        """(columns, magnitude factors) of a case."""
        if kind == "channel":
            return [self.chan], [1.0]
        if kind == "block":
            return self.pos[:, 0].tolist(), [1.0] * self.pos.shape[0]
        blocks = [self.one] if kind in ("one", "mixed-one") else range(self.pos.shape[0])
        if kind.startswith("mixed"):
            f = [1.0, 0.1, 0.01, 0.001]
            return [int(self.pos[b, i]) for b in blocks for i in range(4)], f * len(list(blocks))
        return [int(self.pos[b, i]) for b in blocks for i in range(count)], [1.0] * (count * len(list(blocks)))


def apply_case(x: np.ndarray, layout: Layout, kind: str, count: int, mag: float) -> np.ndarray:
    """x (fp32, N(0,1)-like, last axis N) with the case's outliers of
    magnitude `mag` (times the case's factors), alternating in sign."""
    x = np.array(x, dtype=np.float32, copy=True)
    cols, f = layout.columns(kind, count)
    sign = np.where(np.arange(len(cols)) % 2 == 0, 1.0, -1.0)
    x[..., cols] = (sign * mag * np.asarray(f)).astype(np.float32)
    return x


KINDS = [("channel", 1), ("block", 1)] + [(s, n) for s in ("one", "all") for n in (2, 3, 4, 6)] + \
        [("mixed-one", 4), ("mixed-all", 4)]
MAGS = (1e3, 1e4, 1e5)
CASES = [(k, n, m) for (k, n) in KINDS for m in MAGS]
