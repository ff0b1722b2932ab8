"""Seeded synthetic inputs for tests and benchmarks.

A counter-based generator (SplitMix64 finalizer over (seed, stream, index)) so
any element can be regenerated independently and every run draws the same
data.  Normal deviates use the Box-Muller transform in float64, then round to
float32.  The reference's own Tensor::randn is unseeded
(src/tensor.cpp:136-153) and is never used for parity data.

Seeds follow the benchmark plan: 0x5EED0000 + config index, with sub-streams
STREAM_W, STREAM_X and STREAM_BIAS for weights, activations and bias, and
STREAM_W2 / STREAM_BIAS2 for the second (up) projection of a gated MLP.
"""
from __future__ import annotations

import numpy as np

STREAM_W, STREAM_X, STREAM_BIAS = 0, 1, 2
STREAM_W2, STREAM_BIAS2 = 3, 4
BASE_SEED = 0x5EED0000

_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def _mix(z: np.ndarray) -> np.ndarray:
    z = z.copy()
    z ^= z >> np.uint64(30)
    z *= _M1
    z ^= z >> np.uint64(27)
    z *= _M2
    z ^= z >> np.uint64(31)
    return z


def _key(seed: int, stream: int) -> np.uint64:
    with np.errstate(over="ignore"):
        k = _mix(np.array([(seed & 0xFFFFFFFF) << 16 | (stream & 0xFFFF)], dtype=np.uint64))[0]
    return k


def uniform_u64(n: int, seed: int, stream: int, offset: int = 0) -> np.ndarray:
    idx = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(idx * _GOLDEN + _key(seed, stream))


def normal(shape, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """float32 N(mean, std) array of `shape`, element i drawn from counters 2i, 2i+1."""
    n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    chunk = 1 << 22
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        u = uniform_u64(2 * m, seed, stream, 2 * s)
        a = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)  # (0, 1]
        b = (u[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)  # [0, 1)
        z = np.sqrt(-2.0 * np.log(a)) * np.cos(2.0 * np.pi * b)
        out[s : s + m] = (mean + std * z).astype(np.float32)
    return out.reshape(shape)


def config_seed(index: int) -> int:
    return BASE_SEED + index
