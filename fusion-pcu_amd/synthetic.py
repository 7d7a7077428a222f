"""Seeded synthetic inputs for the BASELINE configurations (no datasets exist offline).

Generator: SplitMix64 with a per-tensor seed; element i uses the (i+1)-th state.
  uniform[-1, 1): f32 (u >> 40) * 2^-23 - 1, f64 (u >> 11) * 2^-52 - 1 (both exact)
  normal(0, s):   Box-Muller in binary64 from two draws, rounded once to the dtype
  xavier-uniform: uniform[-1, 1) times sqrt(6 / (fan_in + fan_out)), in binary64,
                  rounded once to the dtype
The same host arrays feed the CPU oracle and the GPU.
"""
from __future__ import annotations

import concurrent.futures
import os

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _fill(n: int, fn, dtype) -> np.ndarray:
    """Chunks are independent (element i depends only on i), so they fill in parallel;
    numpy's ufuncs release the GIL."""
    out = np.empty(n, dtype=dtype)

    def work(start):
        stop = min(n, start + _CHUNK)
        out[start:stop] = fn(start, stop - start)

    starts = list(range(0, n, _CHUNK))
    if len(starts) <= 1:
        for s in starts:
            work(s)
        return out
    workers = min(len(starts), max(1, min(16, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(work, starts))
    return out


def uniform(seed: int, shape, dtype=np.float32) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))
    if np.dtype(dtype) == np.float32:
        fn = lambda o, m: ((splitmix64(seed, m, o) >> np.uint64(40)).astype(np.float64) * 2.0 ** -23 - 1.0).astype(np.float32)
    else:
        fn = lambda o, m: (splitmix64(seed, m, o) >> np.uint64(11)).astype(np.float64) * 2.0 ** -52 - 1.0
    return _fill(n, fn, dtype).reshape(shape)


def normal(seed: int, shape, std=1.0, dtype=np.float32) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))

    def fn(o, m):
        u = splitmix64(seed, 2 * m, 2 * o)
        u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
        u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2) * float(std)
        return z.astype(dtype)

    return _fill(n, fn, dtype).reshape(shape)


def xavier_uniform(seed: int, fan_in: int, fan_out: int, dtype=np.float32) -> np.ndarray:
    bound = np.sqrt(6.0 / (fan_in + fan_out))
    n = fan_in * fan_out

    def fn(o, m):
        u = (splitmix64(seed, m, o) >> np.uint64(11)).astype(np.float64) * 2.0 ** -52 - 1.0
        return (u * bound).astype(dtype)

    return _fill(n, fn, dtype).reshape(fan_in, fan_out)


def sample_indices(seed: int, population: int, count: int) -> np.ndarray:
    """`count` distinct indices of [0, population), seeded (sampling without replacement)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return np.sort(rng.choice(population, size=count, replace=False))
