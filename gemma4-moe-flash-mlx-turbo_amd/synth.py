"""Seeded synthetic K/V/q for the benchmark workloads (host-side, numpy).

Generator: SplitMix64 over counter i (state = seed + (i+1) * golden gamma),
uniforms u = ((z >> 11) + 1) * 2^-53 in (0, 1], Box-Muller in f64, then
f64 -> f32 -> bf16 (round to nearest even). Outlier channels: 4 channels per
KV head, drawn without replacement from a seeded permutation, scaled x20 on
K, V and on the query heads that read that KV head.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n outputs of SplitMix64 seeded with `seed`, starting at draw `offset`."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    z = splitmix64(seed, n, offset)
    return ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)


def normal(seed: int, shape, offset: int = 0) -> np.ndarray:
    n = int(np.prod(shape))
    u = uniform(seed, 2 * n, 2 * offset)
    z = np.sqrt(-2.0 * np.log(u[0::2])) * np.cos(2.0 * np.pi * u[1::2])
    return z.reshape(shape)


def student_t3(seed: int, shape, offset: int = 0) -> np.ndarray:
    """Student-t with 3 degrees of freedom: Z / sqrt(chi2_3 / 3)."""
    n = int(np.prod(shape))
    z = normal(seed, (4 * n,), 4 * offset)
    num = z[0::4]
    chi2 = z[1::4] ** 2 + z[2::4] ** 2 + z[3::4] ** 2
    return (num / np.sqrt(chi2 / 3.0)).reshape(shape)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def outlier_channels(seed: int, n_heads: int, head_dim: int, count: int = 4) -> np.ndarray:
    """[n_heads, count] channel indices (seeded permutation per head)."""
    out = np.empty((n_heads, count), dtype=np.int64)
    for h in range(n_heads):
        keys = splitmix64(seed ^ 0x0C7A11E5, head_dim, h * head_dim)
        out[h] = np.sort(np.argsort(keys, kind="stable")[:count])
    return out


def kv_rows(seed: int, n_tokens: int, n_kv_heads: int, head_dim: int, outliers: np.ndarray | None,
            dist: str = "normal", offset: int = 0) -> np.ndarray:
    """bf16 bit patterns [n_tokens, n_kv_heads, head_dim] for token range
    [offset, offset + n_tokens) of one seeded stream."""
    shape = (n_tokens, n_kv_heads, head_dim)
    off = offset * n_kv_heads * head_dim
    x = student_t3(seed, shape, off) if dist == "t3" else normal(seed, shape, off)
    if outliers is not None:
        for h in range(n_kv_heads):
            x[:, h, outliers[h]] *= 20.0
    return f32_to_bf16_bits(x.astype(np.float32))


def q_rows(seed: int, n_q_heads: int, n_kv_heads: int, head_dim: int, outliers: np.ndarray | None,
           offset: int = 0, batch: int | None = None) -> np.ndarray:
    shape = (n_q_heads, head_dim) if batch is None else (batch, n_q_heads, head_dim)
    x = normal(seed, shape, offset * n_q_heads * head_dim)
    if outliers is not None:
        rep = n_q_heads // n_kv_heads
        for h in range(n_q_heads):
            x[..., h, outliers[h // rep]] *= 20.0
    return f32_to_bf16_bits(x.astype(np.float32))
