"""Seeded synthetic inputs shared by the tests, the oracle and the GPU generator.

Element i of stream `seed`: SplitMix64 at counter i (state = seed + (i+1)*gamma),
uniform u_i = (z >> 11) * 2^-53; pair k uses (u_2k, u_2k+1) in Box-Muller
    r = sqrt(-2 ln(1 - u_2k)),  th = 2 pi u_2k+1,
    x_2k = r cos th,  x_2k+1 = r sin th        (all in f64)
then y = x * scale + shift in f64, rounded to f32, then to bf16 (round to
nearest even). libvallmo_attn's vm_fill_normal_bf16 implements the same stream
on the GPU (checked bit-for-bit in tests/test_gpu_rows.py).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(seed: int, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx.astype(np.uint64) + np.uint64(1)) * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def f32_to_bf16(x) -> np.ndarray:
    """Round fp32 to bf16 bits, nearest-even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    with np.errstate(over="ignore"):
        r = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return (r >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_f32(n: int, seed: int, scale: float = 1.0, shift: float = 0.0) -> np.ndarray:
    """The f32 values (before bf16 rounding) of stream `seed`, n elements."""
    pairs = (n + 1) // 2
    k = np.arange(pairs, dtype=np.uint64)
    u1 = (_splitmix64(seed, 2 * k) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    u2 = (_splitmix64(seed, 2 * k + 1) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    th = 6.283185307179586 * u2
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(th)
    out[1::2] = r * np.sin(th)
    out = out[:n] * float(np.float32(scale)) + float(np.float32(shift))
    return out.astype(np.float32)


def normal_bf16(shape, seed: int, scale: float = 1.0, shift: float = 0.0) -> np.ndarray:
    """bf16 bits of shape `shape` drawn from stream `seed`."""
    n = int(np.prod(shape))
    return f32_to_bf16(normal_f32(n, seed, scale, shift)).reshape(shape)
