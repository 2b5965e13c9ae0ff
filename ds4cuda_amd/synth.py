"""Seeded synthetic inputs shared by tests, bench and the CPU baseline.

splitmix64(seed) stream -> Box-Muller in fp64 -> fp32, then RNE to bf16 where
a config asks for bf16. Stream k of a seed uses seed*1_000_003 + k as its
splitmix64 state, so independent tensors of one config never overlap.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(state: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 started at `state` (the state is advanced
    before each output, as in the published algorithm)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(state & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, stream: int, n: int, std: float = 1.0) -> np.ndarray:
    """n fp32 samples of N(0, std^2): Box-Muller on pairs of splitmix64
    outputs, u in (0, 1] from the top 53 bits."""
    m = (n + 1) // 2
    z = splitmix64(seed * 1_000_003 + stream, 2 * m)
    u = ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (out[:n] * std).astype(np.float32)


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    z = splitmix64(seed * 1_000_003 + stream, n)
    return (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    return ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << np.uint32(16)).view(np.float32)


def kv_rows(seed: int, stream: int, n_rows: int, head_dim: int = 512,
            outlier_frac: float = 0.0, outlier_scale: float = 8.0) -> np.ndarray:
    """KV rows ~N(0,1) fp32; a fraction of rows (uniform < outlier_frac) is
    multiplied by outlier_scale to stress the FP8 scale range."""
    x = normal(seed, stream, n_rows * head_dim).reshape(n_rows, head_dim)
    if outlier_frac > 0:
        sel = uniform(seed, stream + 7919, n_rows) < outlier_frac
        x[sel] *= outlier_scale
    return x
