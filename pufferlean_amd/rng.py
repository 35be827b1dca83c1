"""Seeded input generation with the reference's splitmix64 (Puffer/RL/Train.lean:18-28).

A stream started at seed ``s`` yields words mix(s + i*G) for i = 1, 2, ... (G the golden gamma),
so n draws are computed at once. ``randf`` is the reference's ``randF lo hi`` (Exe/Puffer.lean:65-67);
normals use Box-Muller on two consecutive draws; Bernoulli(p) is ``uniform01 < p``.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def words(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Words number start+1 .. start+n of the splitmix64 stream seeded with ``seed``."""
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def state_after(seed: int, n: int) -> int:
    """Generator state after n draws (the state advances by G per draw)."""
    return (seed + n * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF


def uniform01(w: np.ndarray) -> np.ndarray:
    return (w >> np.uint64(11)).astype(np.float64) / 9007199254740992.0


def randf(seed: int, n: int, lo: float, hi: float, start: int = 0) -> np.ndarray:
    return lo + (hi - lo) * uniform01(words(seed, n, start))


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    u = uniform01(words(seed, 2 * n))
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return mean + std * z


def bernoulli(seed: int, n: int, p: float) -> np.ndarray:
    return (uniform01(words(seed, n)) < p).astype(np.float64)


def randint(seed: int, n: int, k: int) -> np.ndarray:
    """Uniform integers in [0, k) as floor(k * u), as the reference draws actions."""
    return np.floor(k * uniform01(words(seed, n))).astype(np.int64)


def seed_for(config: int, tensor: int) -> int:
    """Per-(config, tensor) seed of the synthetic workloads."""
    return 0xB5E10000 + config * 16 + tensor
