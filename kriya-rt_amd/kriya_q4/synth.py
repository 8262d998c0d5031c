"""Seeded synthetic inputs for the five benchmark configurations.

Generator (fixed so that any host regenerates byte-identical inputs):
  SplitMix64: output i (i = 1, 2, ...) of stream `seed` is mix64(seed + i * 0x9E3779B97F4A7C15).
  uniform(u)  = (u >> 11) * 2**-53
  normal      = sqrt(-2 ln(1 - u1)) * cos(2 pi u2) from two consecutive outputs, in float64.
  bf16        = round-to-nearest-even of the float32 value (crates/kriya-core/src/quantizer.rs:19-24).
Q4_G64 weights with the distribution of the benchmark configs:
  nibbles     = the raw bits of stream (seed, 1): u64 output i gives planar words 2i (low half)
                and 2i+1 (high half), so every nibble is uniform on 0..15;
  scales      = bf16(|N(0, 0.02)| + 1e-3) from stream (seed, 2);
  biases      = bf16(-8 * scale), exact.
Per config c, tensor t uses seed c * 1000 + t.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def mix64(v: int) -> int:
    return int(_mix(np.array([v], dtype=np.uint64))[0])


def substream(seed: int, tag: int) -> int:
    return mix64((seed * 0x100 + tag) & 0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint64)
    base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        for lo in range(0, count, _CHUNK):
            hi = min(count, lo + _CHUNK)
            i = np.arange(lo + 1, hi + 1, dtype=np.uint64)
            out[lo:hi] = _mix(base + i * _GAMMA)
    return out


def uniform(u: np.ndarray) -> np.ndarray:
    return (u >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, count: int) -> np.ndarray:
    u = splitmix64(seed, 2 * count).reshape(count, 2)
    r = np.sqrt(-2.0 * np.log1p(-uniform(u[:, 0])))
    return r * np.cos(2.0 * np.pi * uniform(u[:, 1]))


def f32_to_bf16_bits(a) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    """bf16 bits of N(0, std^2), shape `shape` (uint16)."""
    count = int(np.prod(shape))
    return f32_to_bf16_bits((normal(substream(seed, 3), count) * std).astype(np.float32)).reshape(shape)


def f32_normal(shape, seed: int) -> np.ndarray:
    count = int(np.prod(shape))
    return normal(substream(seed, 4), count).astype(np.float32).reshape(shape)


def q4_weight(n: int, k: int, seed: int):
    """(qw uint32 [n, k/8], scales uint16 [n, k/64], biases uint16 [n, k/64])."""
    assert k % 64 == 0
    qw = splitmix64(substream(seed, 1), n * k // 16).view(np.uint32).reshape(n, k // 8)
    z = normal(substream(seed, 2), n * k // 64)
    scales = f32_to_bf16_bits((np.abs(0.02 * z) + 1e-3).astype(np.float32)).reshape(n, k // 64)
    biases = f32_to_bf16_bits(-8.0 * bf16_bits_to_f32(scales))
    return qw, scales, biases


# ---- shapes of the benchmark configurations (configs 0-4) ----
HIDDEN, INTER, VOCAB = 2048, 11008, 151936
Q_DIM, KV_DIM = 2048, 256
MOE_EXPERTS, MOE_TOPK, MOE_INTER = 60, 4, 1408
