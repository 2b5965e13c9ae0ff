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


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= (1 << 63) else v


def normal_device(seed: int, stream: int, n: int, device, std: float = 1.0, chunk: int = 1 << 24):
    """The same samples as normal(seed, stream, n, std), generated on `device`
    with torch integer ops (64-bit wrapping arithmetic, logical shifts by
    masking), so large inputs need no host generation or upload. The fp64
    log / cos of the device may differ from the host's in the last fp64 bit,
    which after the fp32 rounding changes a value only in rare ties."""
    import torch
    m = (n + 1) // 2
    state = _signed((seed * 1_000_003 + stream) & 0xFFFFFFFFFFFFFFFF)
    gold, m1, m2 = (_signed(int(c)) for c in (_GOLDEN, _M1, _M2))
    out = torch.empty(2 * m, dtype=torch.float32, device=device)

    def lsr(z, k):
        return (z >> k) & ((1 << (64 - k)) - 1)

    for p0 in range(0, m, chunk):
        p1 = min(m, p0 + chunk)
        i = torch.arange(2 * p0 + 1, 2 * p1 + 1, dtype=torch.int64, device=device)
        z = state + i * gold
        z = (z ^ lsr(z, 30)) * m1
        z = (z ^ lsr(z, 27)) * m2
        z = z ^ lsr(z, 31)
        u = (lsr(z, 11).to(torch.float64) + 1.0) * (1.0 / 9007199254740992.0)
        u1, u2 = u[0::2], u[1::2]
        r = torch.sqrt(-2.0 * torch.log(u1))
        seg = torch.empty(2 * (p1 - p0), dtype=torch.float64, device=device)
        seg[0::2] = r * torch.cos(2.0 * torch.pi * u2)
        seg[1::2] = r * torch.sin(2.0 * torch.pi * u2)
        out[2 * p0:2 * p1] = (seg * std).to(torch.float32)
    return out[:n]


def uniform_device(seed: int, stream: int, n: int, device):
    """uniform(seed, stream, n) generated on `device` (fp64)."""
    import torch
    state = _signed((seed * 1_000_003 + stream) & 0xFFFFFFFFFFFFFFFF)
    gold, m1, m2 = (_signed(int(c)) for c in (_GOLDEN, _M1, _M2))
    lsr = lambda z, k: (z >> k) & ((1 << (64 - k)) - 1)
    i = torch.arange(1, n + 1, dtype=torch.int64, device=device)
    z = state + i * gold
    z = (z ^ lsr(z, 30)) * m1
    z = (z ^ lsr(z, 27)) * m2
    z = z ^ lsr(z, 31)
    return lsr(z, 11).to(torch.float64) * (1.0 / 9007199254740992.0)


def kv_rows_device(seed: int, stream: int, n_rows: int, device, head_dim: int = 512,
                   outlier_frac: float = 0.0, outlier_scale: float = 8.0):
    """kv_rows() generated on `device`."""
    x = normal_device(seed, stream, n_rows * head_dim, device).reshape(n_rows, head_dim)
    if outlier_frac > 0:
        sel = uniform_device(seed, stream + 7919, n_rows, device) < outlier_frac
        x[sel] *= outlier_scale
    return x
