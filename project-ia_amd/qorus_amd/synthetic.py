"""Seeded synthetic Q4_0 data and model files (the generator the BASELINE
configs describe): nibbles uniform in 0..15, block scale |N(0,1)| * 0.02 as
float32, activations / embeddings / KV entries N(0,1) float32."""
from __future__ import annotations

import zlib

import numpy as np

from .model_file import QorusHeader, write_qorus_v3


def rng_for(seed: int, *stream) -> np.random.Generator:
    return np.random.default_rng([int(seed)] + [int(s) for s in stream])


def gen_q4(M: int, N: int, rng: np.random.Generator) -> np.ndarray:
    """Q4_0 matrix [M, N] as uint8 [M, N/32*20] (AoS 20-byte blocks)."""
    if N % 32:
        raise ValueError("N must be a multiple of 32")
    nblk = N // 32
    blocks = np.empty((M, nblk, 20), dtype=np.uint8)
    blocks[:, :, :16] = rng.integers(0, 256, size=(M, nblk, 16), dtype=np.uint8)
    sc = (np.abs(rng.standard_normal((M, nblk), dtype=np.float32)) * np.float32(0.02)).astype(np.float32)
    blocks[:, :, 16:] = sc.view(np.uint8).reshape(M, nblk, 4)
    return blocks.reshape(M, nblk * 20)


def gen_f32(n, rng: np.random.Generator) -> np.ndarray:
    return rng.standard_normal(n, dtype=np.float32)


def write_synthetic_model(path, h: QorusHeader, seed: int, norm_jitter: float = 0.1) -> int:
    """A random-init Llama-shaped v3 model: Q4_0 matrices as above, fp32
    embeddings N(0,1), RMSNorm weights 1 + norm_jitter * N(0,1)."""

    def get(name, kind, shape):
        rng = rng_for(seed, zlib.crc32(name.encode()))
        if kind == "q4":
            return gen_q4(shape[0], shape[1], rng)
        if name.endswith("norm"):
            return (1.0 + norm_jitter * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
        return rng.standard_normal(shape, dtype=np.float32)

    return write_qorus_v3(path, h, get)
