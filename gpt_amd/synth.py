"""Deterministic synthetic inputs for the attention benchmarks and tests.

A counter-based generator (splitmix64 of seed + (i+1) * golden-gamma) feeds a
Box-Muller transform, vectorised in numpy, so every host produces the same
fp32 tensors for a given seed without depending on a library's RNG.

Configurations follow the benchmark definitions (BASELINE.json ``configs``):
Q/K/V ~ N(0, 1) (times a per-layer factor U[0.5, 2] for the 12-layer
workload), upstream gradient dO ~ N(0, sigma=1e-3), seed 1234 + config index
(+ layer for the 12-layer workload).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset .. offset+n-1 of the splitmix64 stream seeded with `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """U[0, 1) doubles from the top 53 bits."""
    return (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, std: float = 1.0, chunk: int = 1 << 22) -> np.ndarray:
    """fp32 N(0, std^2) array: Box-Muller (cos branch) on stream pairs (2i, 2i+1)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        u = uniform(seed, 2 * m, 2 * s).reshape(m, 2)
        u1 = 1.0 - u[:, 0]  # (0, 1]
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u[:, 1])
        out[s:s + m] = (z * std).astype(np.float32)
    return out.reshape(shape)


def qkv(B: int, T: int, C: int, seed: int, scale: float = 1.0) -> np.ndarray:
    """Packed qkv [B, T, 3C], iid N(0, scale^2)."""
    x = normal(seed, (B, T, 3 * C))
    if scale != 1.0:
        x *= np.float32(scale)
    return x


def grad_out(B: int, T: int, C: int, seed: int, std: float = 1e-3) -> np.ndarray:
    """Upstream gradient dO [B, T, C], iid N(0, std^2); stream offset by 2^40."""
    return normal(seed + (1 << 40), (B, T, C), std=std)


def layer_scales(n_layers: int, seed: int) -> np.ndarray:
    """Per-layer factors U[0.5, 2] for the multi-layer workload."""
    return 0.5 + 1.5 * uniform(seed + (1 << 41), n_layers)
