"""Deterministic, platform-independent synthetic data for the LFM2.5 path.

Every tensor is drawn from its own SplitMix64 stream keyed by (seed, name):
    key      = mix(seed XOR fnv1a64(name))
    word_i   = mix(key + (i + 1) * GOLDEN)          (the SplitMix64 sequence)
    u_i      = ((word_i >> 11) + 1) * 2**-53         in (0, 1]
Normal values use Box-Muller on consecutive pairs (u_2j, u_2j+1) in float64:
    r = sqrt(-2 ln u_2j), n_2j = r cos(2 pi u_2j+1), n_2j+1 = r sin(2 pi u_2j+1)
and value = mean + std * n, rounded to float32 then to BF16 (nearest even).
Uniform integers in [0, 2**k) take the top k bits of word_i.

The same (seed, name) always yields the same bits, independent of torch or
numpy random state, so the GPU path and the CPU oracle see identical inputs.
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .bf16 import f32_to_bf16_bits

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 20


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _mix_scalar(x: int) -> int:
    with np.errstate(over="ignore"):
        return int(_mix(np.array([x & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))[0])


def fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode("utf-8"):
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_key(seed: int, name: str) -> int:
    return _mix_scalar((int(seed) & 0xFFFFFFFFFFFFFFFF) ^ fnv1a64(name))


def words(key: int, start: int, count: int) -> np.ndarray:
    """word_i for i in [start, start + count) of the stream `key`."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(np.uint64(key) + i * GOLDEN)


def _normal_chunk(key: int, start: int, m: int, mean: float, std: float) -> np.ndarray:
    pairs = (m + 1) // 2
    w = words(key, start, 2 * pairs)
    u = ((w >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * (2.0 ** -53)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    theta = (2.0 * np.pi) * u2
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(theta)
    z[1::2] = r * np.sin(theta)
    return f32_to_bf16_bits((mean + std * z[:m]).astype(np.float32))


def normal_bf16(seed: int, name: str, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n BF16 values (uint16 bit patterns) of mean + std * N(0, 1)."""
    key = stream_key(seed, name)
    out = np.empty(n, dtype=np.uint16)
    starts = range(0, n, _CHUNK)  # _CHUNK is even: pairs never straddle chunks

    def fill(start):
        m = min(_CHUNK, n - start)
        out[start:start + m] = _normal_chunk(key, start, m, mean, std)

    if n <= _CHUNK:
        fill(0)
    else:
        with ThreadPoolExecutor(max_workers=_workers()) as pool:
            list(pool.map(fill, starts))
    return out


def _workers() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def uniform_ints(seed: int, name: str, n: int, bits: int) -> np.ndarray:
    """n integers uniform in [0, 2**bits), as int32 (bits <= 31) or int64."""
    if not 1 <= bits <= 63:
        raise ValueError("bits must be in [1, 63]")
    w = words(stream_key(seed, name), 0, n)
    v = (w >> np.uint64(64 - bits)).astype(np.int64)
    return v.astype(np.int32) if bits <= 31 else v
