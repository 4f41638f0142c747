"""Seeded synthetic operands for the quantized linear path.

Generator: numpy PCG64 (`numpy.random.default_rng`), standard normals in
float32, rounded to bf16 with round-to-nearest-even on the host, so every
run (CPU oracle, GPU, benchmark) sees the same bits for a given seed.

Activations X [M, K] ~ N(0, 1); round(0.005 * K) outlier channels, chosen by a
seeded permutation, are multiplied by 20 before the bf16 cast.
Weights W [N, K] ~ N(0, 0.02).
X uses default_rng(seed); W uses default_rng(seed + 7919).
"""
from __future__ import annotations

import numpy as np

# Decoder-layer projections of the BASELINE configs: name -> (N, K).
PROJECTIONS = {
    "qkv": (4096, 2048),
    "o_proj": (2048, 2048),
    "gate_up": (12288, 2048),
    "down": (2048, 6144),
}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def outlier_channels(K: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    count = int(round(0.005 * K))
    return np.sort(rng.permutation(K)[:count])


def activations(M: int, K: int, seed: int = 0) -> np.ndarray:
    """bf16 bits [M, K]."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    count = int(round(0.005 * K))
    channels = rng.permutation(K)[:count]
    x[:, channels] *= 20.0
    return f32_to_bf16_bits(x)


def weights(N: int, K: int, seed: int = 0) -> np.ndarray:
    """bf16 bits [N, K]."""
    rng = np.random.default_rng(seed + 7919)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    return f32_to_bf16_bits(w)
