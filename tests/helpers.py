"""Seeded inputs and block builders shared by the tests."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def xorshift_noise(n: int, seed: int) -> np.ndarray:
    """Deterministic floats in [-1, 1): the generator of crates/ggml-sys/tests/iqk_kernels.rs:39-48
    (xorshift64 13/7/17, top 24 bits as a fraction)."""
    out = np.empty(n, dtype=np.float32)
    s = seed & 0xFFFFFFFFFFFFFFFF
    mask = 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        out[i] = np.float32((s >> 40) / float(1 << 23) - 1.0)
    return out


def normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def random_blocks(ty: int, nblocks: int, seed: int) -> np.ndarray:
    """Random valid blocks: every bit pattern of the quant and scale fields, with fp16 d (and dmin)
    drawn from a sane positive range so sums stay finite."""
    rng = np.random.default_rng(seed)
    dt = O.BLOCK_DTYPE[ty]
    raw = rng.integers(0, 256, size=nblocks * dt.itemsize, dtype=np.uint8)
    b = raw.view(dt)
    b["d"] = rng.uniform(1e-3, 1e-2, size=nblocks).astype(np.float16).view(np.uint16)
    if ty == O.TYPE_Q4_K:
        b["dmin"] = rng.uniform(5e-4, 5e-3, size=nblocks).astype(np.float16).view(np.uint16)
    return raw


def pack_q4_K_scales(sc, m) -> np.ndarray:
    """The 12-byte scale field for eight 6-bit scales and mins (inverse of the unpack in
    patches/0002-iqk-avx512-q4k-q6k-decode.patch:371-380)."""
    s = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def half_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])
