"""The `seeded` initial-value generator (reference: runtime/initgen.py:1-58), vectorised with numpy.

Draw j of seed s is SplitMix64 at counter j: z = s + (j+1)*0x9E3779B97F4A7C15, then the SplitMix64 finaliser;
u = (z >> 40) * 2^-24. Element i takes `draws` consecutive draws; every step is one float32 operation:
uniform: value = (u - 0.5) * f32(2*scale); normal: value = (((u0+u1) + (u2+u3)) - 2) * f32(scale*sqrt(3)).
"""
from __future__ import annotations

import math
import struct

import numpy as np

GOLDEN = 0x9E3779B97F4A7C15


def _f32(x):
    return struct.unpack('<f', struct.pack('<f', x))[0]


def params(dist: str, scale: float):
    """(draws, bias, coef) written into the bundle metadata."""
    if dist == 'uniform':
        return 1, 0.5, _f32(2.0 * scale)
    if dist == 'normal':
        return 4, 2.0, _f32(scale * math.sqrt(3.0))
    raise ValueError(f'unknown dist {dist!r}')


def _u(seed: int, j: np.ndarray) -> np.ndarray:
    z = np.uint64(seed) + (j + np.uint64(1)) * np.uint64(GOLDEN)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    z = z ^ (z >> np.uint64(31))
    return (z >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)


def seeded(seed: int, n: int, draws: int, bias: float, coef: float) -> np.ndarray:
    with np.errstate(over='ignore'):
        i = np.arange(n, dtype=np.uint64)
        if draws == 1:
            acc = _u(seed, i)
        else:
            j = i * np.uint64(draws)
            acc = (_u(seed, j) + _u(seed, j + np.uint64(1))) + (_u(seed, j + np.uint64(2)) + _u(seed, j + np.uint64(3)))
    return (acc - np.float32(bias)) * np.float32(coef)
