"""Seeded N(0,1) synthetic inputs shared by the tests, the smoke check and the benchmark.

The reference has no tensor generator for these workloads, so this module defines one that any
host (Python here, Java later) can reproduce bit for bit:

* a counter-based SplitMix64 stream: word ``i`` of stream ``key`` is
  ``mix(key + (i + 1) * 0x9E3779B97F4A7C15)`` with the SplitMix64 finaliser
  (constants 0xBF58476D1CE4E5B9, 0x94D049BB133111EB; shifts 30, 27, 31);
* ``key = mix(seed * 0x100000001B3 ^ fnv1a64(tag))`` so every named tensor (``"q/layer3"``…)
  has its own stream;
* Box-Muller in float64 on words ``2j`` and ``2j+1``: ``u1 = ((w0 >> 11) + 1) * 2^-53``,
  ``u2 = (w1 >> 11) * 2^-53``, ``z = sqrt(-2 ln u1) * cos(2 pi u2)``, rounded to float32.
"""

from __future__ import annotations

import os

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    z ^= z >> np.uint64(30)
    z *= _M1
    z ^= z >> np.uint64(27)
    z *= _M2
    z ^= z >> np.uint64(31)
    return z


def _fnv1a64(tag: str) -> int:
    h = 0xCBF29CE484222325
    for b in tag.encode("utf-8"):
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_key(seed: int, tag: str) -> np.uint64:
    base = ((seed * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF) ^ _fnv1a64(tag)
    return _mix(np.array([base], dtype=np.uint64))[0]


def words(seed: int, tag: str, count: int, offset: int = 0) -> np.ndarray:
    key = stream_key(seed, tag)
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        return _mix(key + idx * _GOLDEN)


_CHUNK = 1 << 20  # values per chunk when a large array is generated on several threads


def _normal_into(out: np.ndarray, key: np.uint64, start: int) -> None:
    """Values start .. start + out.size of the stream with key ``key``, written into ``out``."""
    n = out.size
    with np.errstate(over="ignore"):
        idx = np.arange(2 * start + 1, 2 * (start + n) + 1, dtype=np.uint64)
        w = _mix(key + idx * _GOLDEN)
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    out[:] = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def normal(seed: int, tag: str, shape) -> np.ndarray:
    """float32 N(0,1) array of ``shape`` from stream (seed, tag). Large arrays are produced in
    chunks on up to 16 threads (numpy releases the GIL); every value depends only on its index, so
    the result is the same as one pass."""
    n = int(np.prod(shape)) if np.ndim(shape) else int(shape)
    key = stream_key(seed, tag)
    out = np.empty(n, np.float32)
    if n <= _CHUNK:
        _normal_into(out, key, 0)
        return out.reshape(shape)
    from concurrent.futures import ThreadPoolExecutor
    starts = range(0, n, _CHUNK)
    workers = max(1, min(16, os.cpu_count() or 1, len(starts)))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(lambda s0: _normal_into(out[s0:s0 + _CHUNK], key, s0), starts))
    return out.reshape(shape)


def uniform_int(seed: int, tag: str, count: int, low: int, high: int) -> np.ndarray:
    """Integers uniform on [low, high] inclusive (rejection-free modulo on 64-bit words)."""
    w = words(seed, tag, count)
    span = np.uint64(high - low + 1)
    return (w % span).astype(np.int64) + low
