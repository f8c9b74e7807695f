"""Seeded synthetic inputs shared by the tests, the benchmark and the CPU
baseline, so that the GPU and the CPU consume identical bytes.

Generator: splitmix64 over a counter, two 53-bit uniforms per pair, then
Box-Muller in double precision, rounded once to fp32.  Seeds are per
(workload, tensor).  Pure numpy; no torch RNG is involved.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np


def _threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n)), 16))

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, n: int) -> np.ndarray:
    """n doubles in [0, 1) (53-bit)."""
    with np.errstate(over="ignore"):
        base = np.uint64(seed) * np.uint64(0x100000001B3)
        ctr = np.arange(n, dtype=np.uint64) + base
    r = _splitmix64(ctr)
    return (r >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def _uniform01_range(seed: int, first: int, count: int) -> np.ndarray:
    """Elements first .. first+count-1 of uniform01(seed, .)."""
    with np.errstate(over="ignore"):
        base = np.uint64(seed) * np.uint64(0x100000001B3) + np.uint64(first)
        ctr = np.arange(count, dtype=np.uint64) + base
    r = _splitmix64(ctr)
    return (r >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


_CHUNK = 1 << 20  # pairs per chunk: keeps the double temporaries cache-sized


def normal(seed: int, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """fp32 N(mean, std^2) via Box-Muller in double (element 2i from the
    cosine and 2i+1 from the sine of pair i), generated chunk by chunk."""
    n = int(np.prod(shape)) if len(shape) else 1
    m = (n + 1) // 2
    out = np.empty(2 * m, np.float32)

    def chunk(p0):
        pc = min(_CHUNK, m - p0)
        u = _uniform01_range(seed, 2 * p0, 2 * pc)
        u1 = 1.0 - u[0::2]  # (0, 1]
        u2 = u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * pc, np.float64)
        z[0::2] = r * np.cos(2.0 * np.pi * u2)
        z[1::2] = r * np.sin(2.0 * np.pi * u2)
        out[2 * p0:2 * (p0 + pc)] = (z * std + mean).astype(np.float32)

    starts = range(0, m, _CHUNK)
    if len(starts) > 1:  # numpy releases the GIL inside these ufuncs
        with ThreadPoolExecutor(min(len(starts), _threads())) as ex:
            list(ex.map(chunk, starts))
    elif m:
        chunk(0)
    return out[:n].reshape(shape)


def uniform(seed: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    return (uniform01(seed, n) * (hi - lo) + lo).astype(np.float32).reshape(shape)
