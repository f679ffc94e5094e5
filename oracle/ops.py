"""NumPy restatement of the reference's decode operators.

Paths are relative to ios_kernels/kernels/ in the reference:
    KL = unsloth__Llama-3.2-1B-Instruct/kernel_metal_f16_20261024-1620/
    KG = google__gemma-4-E2B-it/kernel_metal_f16_20261025-1225/

Every op computes in float64 from its (fp16 / fp32) inputs and returns float64;
the caller decides where values are rounded (model.py rounds at the same points
as the GPU: fp32 activations between ops, fp16 KV cache).

KV caches are in the reference's layout, K and V both [n_kv, max_ctx, hd]
(KL/kernels.metal:10); the GPU library's tiled V layout is a storage detail
the tests convert.
"""

from __future__ import annotations

import math

import numpy as np

F64 = np.float64


def matvec(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[r] = sum_k W[r, k] * x[k] (KL/kernels.metal:106-137; KG/kernels.metal:159-198)."""
    return W.astype(F64) @ np.asarray(x, dtype=F64)


def quantize_q8b32(W: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Block-32 symmetric int8: s = fp16(max|w| / 127); q = clip(rint(w / s), -127, 127),
    the division done in fp32 against the fp16 scale; zero blocks give s = q = 0."""
    M, K = W.shape
    blocks = W.astype(np.float32).reshape(M, K // 32, 32)
    amax = np.max(np.abs(blocks), axis=2)
    s = (amax / np.float32(127)).astype(np.float16)
    q = np.zeros(blocks.shape, dtype=np.int8)
    sf = s.astype(np.float32)
    nz = sf > 0
    r = np.rint(blocks[nz] / sf[nz][:, None])
    q[nz] = np.clip(r, -127, 127).astype(np.int8)
    return q.reshape(M, K), s


def matvec_q8b32(q: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[r] = sum_b s[r, b] * sum_{k in b} q[r, k] * x[k] (integer weights, exact products)."""
    M, K = q.shape
    xb = np.asarray(x, dtype=F64).reshape(K // 32, 32)
    part = np.einsum("mbk,bk->mb", q.reshape(M, K // 32, 32).astype(F64), xb)
    return (part * s.astype(F64)).sum(axis=1)


def gelu_tanh(x):
    """gelu_pytorch_tanh (KG/kernels.metal:26-28)."""
    x = np.asarray(x, dtype=F64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x**3)))


def silu(x):
    """g / (1 + e^-g) (KL/kernels.metal:171)."""
    x = np.asarray(x, dtype=F64)
    return x / (1.0 + np.exp(-x))


def gate_up(Wg, Wu, x, act: str = "gelu_tanh") -> np.ndarray:
    """h = act(Wg.x) * (Wu.x) (KG/kernels.metal:205-234; KL/kernels.metal:144-173)."""
    g, u = matvec(Wg, x), matvec(Wu, x)
    return (gelu_tanh(g) if act == "gelu_tanh" else silu(g)) * u


def gate_up_q8b32(qg, sg, qu, su, x, act: str = "gelu_tanh") -> np.ndarray:
    g, u = matvec_q8b32(qg, sg, x), matvec_q8b32(qu, su, x)
    return (gelu_tanh(g) if act == "gelu_tanh" else silu(g)) * u


def rmsnorm(x, w, eps: float, plus_one: bool = False) -> np.ndarray:
    """y = x * rsqrt(mean(x^2) + eps) * w, per row (KL/kernels.metal:71-96); plus_one
    uses the Gemma (1 + w) weight convention."""
    x = np.asarray(x, dtype=F64)
    w = np.asarray(w, dtype=F64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * ((1.0 + w) if plus_one else w)


def inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """1 / theta^(2i/hd) in double, stored as fp32 (KL/main.swift:92-94, 108)."""
    i = np.arange(head_dim // 2, dtype=F64)
    return (1.0 / theta ** (2.0 * i / head_dim)).astype(np.float32)


def inv_freq_llama3(head_dim: int, theta: float, factor: float, low_freq_factor: float, high_freq_factor: float,
                    original_max_positions: int) -> np.ndarray:
    """Llama-3 frequency scaling of inv_freq, in double, stored as fp32
    (KL/main.swift:96-107): a frequency whose wavelength 2 pi / f is shorter
    than original / high_freq_factor is kept, one longer than
    original / low_freq_factor is divided by factor, and in between the two
    are blended linearly in original / wavelength."""
    i = np.arange(head_dim // 2, dtype=F64)
    f = 1.0 / theta ** (2.0 * i / head_dim)
    wavelen = 2.0 * math.pi / f
    lo_wave = original_max_positions / low_freq_factor
    hi_wave = original_max_positions / high_freq_factor
    t = (original_max_positions / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    blended = (1.0 - t) * f / factor + t * f
    out = np.where(wavelen < hi_wave, f, np.where(wavelen > lo_wave, f / factor, blended))
    return out.astype(np.float32)


def rope(v: np.ndarray, pos: int, invf: np.ndarray) -> np.ndarray:
    """rotate_half RoPE of one head vector: pairs (i, i + hd/2) rotated by
    ang = fp32(pos) * inv_freq[i] (the angle is an fp32 product, as on the
    device), sin/cos and the rotation in fp64 (KL/kernels.metal:199-210)."""
    v = np.asarray(v, dtype=F64)
    half = v.shape[-1] // 2
    ang = (np.float32(pos) * invf.astype(np.float32)).astype(F64)
    c, s = np.cos(ang), np.sin(ang)
    a, b = v[..., :half], v[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def rope_kv(qkv_row: np.ndarray, kcache: np.ndarray, vcache: np.ndarray, invf: np.ndarray, n_heads: int,
            n_kv: int, pos: int) -> np.ndarray:
    """One qkv row [q NH*hd | k NKV*hd | v NKV*hd] at position pos: returns the
    rotated q (fp64) and appends the rotated k and v to the caches, rounded to
    the caches' dtype: fp16 as on the device (KL/kernels.metal:189-224), or
    unrounded into fp64 caches. kcache, vcache [n_kv, ctx, hd]."""
    hd = kcache.shape[2]
    row = np.asarray(qkv_row, dtype=F64)
    q = row[: n_heads * hd].reshape(n_heads, hd)
    k = row[n_heads * hd : (n_heads + n_kv) * hd].reshape(n_kv, hd)
    v = row[(n_heads + n_kv) * hd :].reshape(n_kv, hd)
    qr = rope(q, pos, invf)
    kr = rope(k, pos, invf)
    kcache[:, pos, :] = kr.astype(kcache.dtype)
    vcache[:, pos, :] = v.astype(vcache.dtype)
    return qr.reshape(-1)


def attention(q: np.ndarray, kcache: np.ndarray, vcache: np.ndarray, n_keys: int, n_heads: int,
              scale: float) -> np.ndarray:
    """out[h] = softmax(scale * q[h] . K[kvh, :n]) . V[kvh, :n], kvh = h // (NH / NKV)
    (KL/kernels.metal:235-305, GQA map at :261); fp64 throughout."""
    n_kv, _, hd = kcache.shape
    G = n_heads // n_kv
    qh = np.asarray(q, dtype=F64).reshape(n_heads, hd)
    out = np.empty((n_heads, hd), dtype=F64)
    for h in range(n_heads):
        kvh = h // G
        K = kcache[kvh, :n_keys, :].astype(F64)
        V = vcache[kvh, :n_keys, :].astype(F64)
        s = (K @ qh[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p @ V) / p.sum()
    return out.reshape(-1)


def argmax(logits: np.ndarray) -> int:
    """The reference's scan `if (v > best)` from best = -inf, index 0
    (KL/kernels.metal:317-331): the first maximum (lowest index among ties);
    NaN and -inf are never selected, and a row of nothing else gives 0."""
    v = np.asarray(logits, dtype=np.float64)
    live = v > -np.inf  # False for NaN and -inf
    if not live.any():
        return 0
    return int(np.argmax(np.where(live, v, -np.inf)))


def embed(E: np.ndarray, token: int, scale: float = 1.0) -> np.ndarray:
    """x = float(E[token]) * scale (KL/kernels.metal:31-39; scale sqrt(D) for Gemma,
    KG/main.swift:397)."""
    return E[token].astype(F64) * scale
