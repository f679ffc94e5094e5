"""NumPy restatement of the synthetic-weight generator (mxd_fill_normal).

Element i of tensor (seed, tensor_id):
    key = mix(mix(seed) ^ tensor_id)
    h0 = mix(key + 2i), h1 = mix(key + 2i + 1)        mix = splitmix64 output function
    c  = (sum of the eight 16-bit fields of h0, h1) - 4 * 65535
    v  = fp32(c) * k,  k = fp32(stddev / sqrt(8 * (65536^2 - 1) / 12))
fp16 tensors round v to nearest even. The weights stand in for the reference's
converted HF checkpoints (KL/convert_weights.py:71-89), which need a download.
"""

from __future__ import annotations

import math

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
SIGMA_SUM = math.sqrt(8 * (65536.0 * 65536.0 - 1.0) / 12.0)


def mix(z: np.ndarray) -> np.ndarray:
    """splitmix64 output for state z (uint64 array, wrapping arithmetic)."""
    z = np.asarray(z, dtype=np.uint64) + _GOLDEN
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def mix_int(z: int) -> int:
    """Pure-integer splitmix64 output (independent of NumPy's uint64 ops)."""
    m = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def key_of(seed: int, tensor_id: int) -> int:
    return mix_int(mix_int(seed) ^ tensor_id)


def scale_of(stddev: float) -> np.float32:
    return np.float32(float(np.float32(stddev)) / SIGMA_SUM)


def _sum16(h: np.ndarray) -> np.ndarray:
    f = np.uint64(0xFFFF)
    return ((h & f) + ((h >> np.uint64(16)) & f) + ((h >> np.uint64(32)) & f) + (h >> np.uint64(48))).astype(np.int64)


def normal_f32(n: int, seed: int, tensor_id: int, stddev: float, start: int = 0) -> np.ndarray:
    """Elements [start, start + n) of the tensor, as fp32."""
    with np.errstate(over="ignore"):
        key = np.uint64(key_of(seed, tensor_id))
        i = np.arange(start, start + n, dtype=np.uint64)
        h0 = mix(key + np.uint64(2) * i)
        h1 = mix(key + np.uint64(2) * i + np.uint64(1))
    c = (_sum16(h0) + _sum16(h1) - 4 * 65535).astype(np.float32)
    return c * scale_of(stddev)


def normal(shape, dtype, seed: int, tensor_id: int, stddev: float) -> np.ndarray:
    n = int(np.prod(shape))
    v = normal_f32(n, seed, tensor_id, stddev).reshape(shape)
    return v.astype(dtype)


def normal_int(i: int, seed: int, tensor_id: int, stddev: float) -> float:
    """One element with Python integers only (a third restatement for tests)."""
    key = key_of(seed, tensor_id)
    m = (1 << 64) - 1
    h0, h1 = mix_int((key + 2 * i) & m), mix_int((key + 2 * i + 1) & m)
    c = sum((h >> s) & 0xFFFF for h in (h0, h1) for s in (0, 16, 32, 48)) - 4 * 65535
    return float(np.float32(c) * scale_of(stddev))
