"""Adversarial GEMV/GEMM inputs: activation outliers that meet zero weights.

An outlier channel whose weight nibble is 8 in every row ((8 - 8) * s = 0)
adds nothing to sum_j |W_ij x_j|, so the outputs' condition is set by the
ordinary elements only.  Any representation of x whose precision follows
the largest element of a group (a shared exponent) loses the ordinary
elements' low bits there, and the error statistic exposes it.  The
reference's fp32 FMA order is unaffected (a zero product changes no sum).
"""
from __future__ import annotations

import numpy as np


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


def outlier_columns(N: int, rng: np.random.Generator):
    """(one channel, one column in each 32-element block)."""
    nblk = N // 32
    chan = int(rng.integers(0, N))
    per_block = np.arange(nblk) * 32 + rng.integers(0, 32, size=nblk)
    return chan, per_block


def apply_outliers(x: np.ndarray, kind: str, mag: float, chan: int, per_block) -> np.ndarray:
    """x (fp32, N(0,1)-like) with outliers of magnitude `mag` (random signs)
    on one channel (kind 'channel') or on one column per block ('block')."""
    x = np.array(x, dtype=np.float32, copy=True)
    cols = [chan] if kind == "channel" else list(per_block)
    sign = np.where(np.arange(len(cols)) % 2 == 0, 1.0, -1.0)
    x[..., cols] = (sign * mag).astype(np.float32)
    return x


CASES = [(k, m) for k in ("channel", "block") for m in (1e3, 1e4, 1e5)]
