"""Tolerances and comparison helpers shared by the tests.

The bars (stated once, used everywhere):
  - found_inf, skip decision, loss scale and growth tracker: bit-exact;
  - params / master / exp_avg / exp_avg_sq (fp32): max relative error
    max|a - b| / max|b| per tensor <= 1e-6 (RTOL_STATE);
  - bf16 / fp16 model params: at most 1 unit in the last place (ULP_LOWP);
  - gradient norm: relative error <= 1e-5 (RTOL_NORM).
"""

from __future__ import annotations

import numpy as np

RTOL_STATE = 1e-6
RTOL_NORM = 1e-5
ULP_LOWP = 1


def maxrel(a: np.ndarray, b: np.ndarray) -> float:
    """max |a - b| / max |b| over one tensor (0 when both are all zero)."""
    a64 = np.asarray(a, np.float64).ravel()
    b64 = np.asarray(b, np.float64).ravel()
    if a64.size == 0:
        return 0.0
    d = float(np.max(np.abs(a64 - b64)))
    s = float(np.max(np.abs(b64)))
    return d / s if s > 0 else d


def exact_fraction(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a).ravel()
    b = np.asarray(b).ravel()
    if a.size == 0:
        return 1.0
    return float(np.mean(a.view(np.uint32) == b.view(np.uint32))) if a.dtype == np.float32 else float(np.mean(a == b))


CHUNK = 1 << 24      # elements per piece of the comparisons below (bounds their temporaries)
_POOL = None


def _map(fn, n: int) -> list:
    """fn(start) for the pieces of an n-element comparison, in threads (numpy
    releases the GIL inside these loops) when there is more than one."""
    global _POOL
    starts = range(0, n, CHUNK)
    if len(starts) <= 1:
        return [fn(s) for s in starts]
    if _POOL is None:
        from concurrent.futures import ThreadPoolExecutor

        _POOL = ThreadPoolExecutor(max_workers=16)
    return list(_POOL.map(fn, starts))


def ulp16(a_bits: np.ndarray, b_bits: np.ndarray) -> int:
    """Largest distance in units in the last place between two arrays of
    bf16/fp16 bit patterns (sign-magnitude mapped to a monotone integer line)."""
    def line(h):
        h = np.asarray(h, np.int64) & 0xFFFF
        return np.where(h & 0x8000, -(h & 0x7FFF), h)

    a_bits, b_bits = np.asarray(a_bits).ravel(), np.asarray(b_bits).ravel()

    def piece(s: int) -> int:
        a, b = a_bits[s:s + CHUNK], b_bits[s:s + CHUNK]
        if np.array_equal(a, b):
            return 0
        return int(np.max(np.abs(line(a) - line(b))))

    return max(_map(piece, a_bits.size), default=0)


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Whether two float32 arrays hold the same bit patterns everywhere
    (NaN payloads included), compared piece by piece."""
    a, b = np.asarray(a).ravel(), np.asarray(b).ravel()
    if a.size != b.size:
        return False
    ua, ub = a.view(np.uint32), b.view(np.uint32)
    return all(_map(lambda s: np.array_equal(ua[s:s + CHUNK], ub[s:s + CHUNK]), ua.size))


def rel(a: float, b: float) -> float:
    if a == b:
        return 0.0
    return abs(a - b) / max(abs(b), 1e-300)
