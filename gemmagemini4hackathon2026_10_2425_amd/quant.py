"""int8 block-32 weight converter (the format mxd_matvec_q8b32 reads).

A row of K weights is cut into K/32 blocks along K. Each block stores one fp16
scale s = fp16(max|w| / 127) and 32 int8 values q = clip(rint(w / s), -127, 127)
(round half to even, computed in fp32 against the fp16-rounded scale, so
q * s is the nearest representable dequantised value). An all-zero block has
s = 0 and q = 0. This is a one-off host conversion, like the reference's
convert_weights.py (KL/convert_weights.py:71-89) is for fp16.
"""

from __future__ import annotations

import numpy as np

BLOCK = 32


def quantize_q8b32(W: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """W [M, K] (fp16/fp32) -> (q int8 [M, K], s fp16 [M, K/32])."""
    if W.ndim != 2 or W.shape[1] % BLOCK:
        raise ValueError(f"quantize_q8b32: W must be [M, K] with K % {BLOCK} == 0, got {W.shape}")
    M, K = W.shape
    w = W.astype(np.float32, copy=False).reshape(M, K // BLOCK, BLOCK)
    s16 = (np.abs(w).max(axis=2) / np.float32(127.0)).astype(np.float16)
    sf = s16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(sf > 0, np.rint(w / np.where(sf > 0, sf, np.float32(1.0))), np.float32(0.0))
    q = np.clip(q, -127, 127).astype(np.int8).reshape(M, K)
    return q, s16


def dequantize_q8b32(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    M, K = q.shape
    return (q.reshape(M, K // BLOCK, BLOCK).astype(np.float32) * s.astype(np.float32)[..., None]).reshape(M, K)
