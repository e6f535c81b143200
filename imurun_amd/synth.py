"""Deterministic synthetic inputs: splitmix64 streams and Box-Muller normals.

One generator for every consumer (tests, benchmark, fixtures) so that the
same (seed, shape) gives the same floats on every machine, independent of
numpy's or the C++ library's distribution code.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n outputs of the splitmix64 sequence started at `seed`, skipping `offset`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Uniform doubles in (0, 1]."""
    return ((splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, std: float = 1.0, chunk: int = 1 << 16) -> np.ndarray:
    """float32 N(0, std^2) of the given shape (Box-Muller on pairs of uniforms).
    Chunks are independent (element i uses uniforms 2i, 2i+1), so large
    arrays are filled by a thread pool; the result does not depend on it."""
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n = int(np.prod(shape)) if shape else 1
    out = np.empty(n, np.float32)

    def fill(s: int) -> None:
        m = min(chunk, n - s)
        u = uniform(seed, 2 * m, 2 * s)
        r = np.sqrt(-2.0 * np.log(u[0::2]))
        out[s:s + m] = (r * np.cos(2.0 * np.pi * u[1::2]) * std).astype(np.float32)

    starts = range(0, n, chunk)
    if n > 8 * chunk:
        import concurrent.futures as cf
        import os
        with cf.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
            list(ex.map(fill, starts))
    else:
        for s in starts:
            fill(s)
    return out.reshape(shape)
