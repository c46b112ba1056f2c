"""Deterministic synthetic inputs for the paged KV path.

Every array is drawn from a counter-based splitmix64 stream keyed by
(seed, name), so any slice can be regenerated independently on any machine:

* ``uniform(seed, name, n)``: 53-bit uniforms in [0, 1);
* ``normal(seed, name, n)``: Box-Muller N(0, 1) in float64, rounded to float32;
* ``permutation(seed, name, n)``: Fisher-Yates shuffle of ``range(n)``;
* ``integers(seed, name, n, low, high)``: uniform integers in [low, high].

``std::normal_distribution`` and ``std::uniform_int_distribution`` are avoided
on purpose: their outputs differ between standard libraries.
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _key(seed: int, name: str) -> np.uint64:
    h = 0xCBF29CE484222325
    for byte in name.encode():
        h = ((h ^ byte) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    with np.errstate(over="ignore"):
        return _mix(np.array([(seed * 0x9E3779B97F4A7C15 + h) & 0xFFFFFFFFFFFFFFFF], np.uint64))[0]


def bits(seed: int, name: str, n: int, start: int = 0) -> np.ndarray:
    """Outputs ``start .. start+n-1`` of the splitmix64 stream keyed by (seed, name)."""
    key = _key(seed, name)
    out = np.empty(n, np.uint64)
    with np.errstate(over="ignore"):
        for lo in range(0, n, _CHUNK):
            hi = min(n, lo + _CHUNK)
            i = np.arange(start + lo + 1, start + hi + 1, dtype=np.uint64)
            out[lo:hi] = _mix(key + i * _GOLDEN)
    return out


def uniform(seed: int, name: str, n: int, start: int = 0) -> np.ndarray:
    return (bits(seed, name, n, start) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def _workers() -> int:
    """Host threads for large draws (the stream is counter-based, so chunks
    are independent and the result does not depend on the count)."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return max(1, min(16, cores))


def normal(seed: int, name: str, n: int) -> np.ndarray:
    """N(0, 1) float32 values by Box-Muller over consecutive uniform pairs."""
    out = np.empty(n, np.float32)
    pairs = (n + 1) // 2
    chunk = 1 << 18  # pairs per task

    def fill(lo):
        hi = min(pairs, lo + chunk)
        u = uniform(seed, name, 2 * (hi - lo), 2 * lo)
        radius = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        angle = 2.0 * np.pi * u[1::2]
        block = np.empty(2 * (hi - lo), np.float64)
        block[0::2] = radius * np.cos(angle)
        block[1::2] = radius * np.sin(angle)
        m = min(n, 2 * hi) - 2 * lo
        out[2 * lo : 2 * lo + m] = block[:m]

    starts = range(0, pairs, chunk)
    if len(starts) > 1:
        with ThreadPoolExecutor(_workers()) as pool:
            list(pool.map(fill, starts))
    else:
        for lo in starts:
            fill(lo)
    return out


def integers(seed: int, name: str, n: int, low: int, high: int) -> np.ndarray:
    """Uniform integers in the closed range [low, high]."""
    u = uniform(seed, name, n)
    return (low + np.floor(u * (high - low + 1))).astype(np.int64)


def permutation(seed: int, name: str, n: int) -> np.ndarray:
    """Fisher-Yates shuffle of range(n)."""
    out = np.arange(n, dtype=np.int64)
    if n < 2:
        return out
    u = uniform(seed, name, n - 1)
    js = np.floor(u * np.arange(n, 1, -1, dtype=np.float64)).astype(np.int64)
    for k, i in enumerate(range(n - 1, 0, -1)):
        j = js[k]
        out[i], out[j] = out[j], out[i]
    return out


def signal(n: int, scale: float = 1.0) -> np.ndarray:
    """``scale * sin(i * 0.173f)`` in float32, the deterministic input of the
    reference's attention tests (tests/core/prefill_support.hpp:10-12)."""
    i = np.arange(n, dtype=np.float32)
    return (np.float32(scale) * np.sin(i * np.float32(0.173))).astype(np.float32)
