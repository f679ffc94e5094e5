"""The decode engine, mirroring the reference's Swift Engine
(ios_kernels/kernels/unsloth__Llama-3.2-1B-Instruct/kernel_metal_f16_20261024-1620/
main.swift:152-491): setTokens / token(at:) / prefill / decode(from:count:) /
decodeStreaming over device-resident weights, KV caches and token buffer.

The arithmetic and the step loop live in libmxdecode.so (mxd_engine_*); this
class is the Python handle. Weights are either synthetic (init_random, the
counter-based generator) or uploaded tensor by tensor (upload).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Iterable

import numpy as np

from . import _lib
from ._lib import call


@dataclass(frozen=True)
class ModelShape:
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    vocab: int
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    act: str = "gelu_tanh"
    norm_plus_one: bool = True
    embed_scale_sqrt_dim: bool = True
    tie_embeddings: bool = True  # LM head = the embedding; else a separate lm_head tensor
    # Llama-3 RoPE scaling (factor, low_freq_factor, high_freq_factor,
    # original_max_position_embeddings), or None for plain RoPE
    rope_scaling: tuple | None = None

    def to_c(self) -> _lib.ModelConfig:
        rs = self.rope_scaling or (0.0, 0.0, 0.0, 0)
        return _lib.ModelConfig(
            self.n_layers, self.dim, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn_dim, self.vocab,
            self.rms_eps, self.rope_theta, _lib.MXD_ACT_SILU if self.act == "silu" else _lib.MXD_ACT_GELU_TANH,
            int(self.norm_plus_one), int(self.embed_scale_sqrt_dim), int(not self.tie_embeddings),
            float(rs[0]), float(rs[1]), float(rs[2]), int(rs[3]),
        )

    @property
    def weight_bytes(self) -> int:
        D, F, qkv = self.dim, self.ffn_dim, (self.n_heads + 2 * self.n_kv_heads) * self.head_dim
        per_layer = 2 * (qkv * D + D * self.n_heads * self.head_dim + 3 * F * D) + 2 * 4 * D
        heads = 1 if self.tie_embeddings else 2
        return self.n_layers * per_layer + heads * 2 * self.vocab * D + 4 * D


# The Gemma-2B-shaped model of the decode benchmark: 18 layers, hidden 2048,
# 8 query heads / 1 KV head of dim 256, GeGLU FFN 16384, vocab 256000.
GEMMA_2B = ModelShape(n_layers=18, dim=2048, n_heads=8, n_kv_heads=1, head_dim=256, ffn_dim=16384, vocab=256000)
# The reference's Llama engine model (Llama-3.2-1B-Instruct): 16 layers, hidden
# 2048, 32 query / 8 KV heads of dim 64, SwiGLU 8192, vocab 128256, Llama-3
# RoPE scaling (KL/main.swift:96-107, 172).
LLAMA32_1B = ModelShape(n_layers=16, dim=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn_dim=8192, vocab=128256,
                        rms_eps=1e-5, rope_theta=500000.0, act="silu", norm_plus_one=False,
                        embed_scale_sqrt_dim=False, tie_embeddings=True, rope_scaling=(32.0, 1.0, 4.0, 8192))


class Engine:
    """Device-resident greedy decoder. Token t of a run is written by the GPU
    into tokens[t + 1]; decode() queues all steps without a host sync."""

    def __init__(self, shape: ModelShape, max_ctx: int = 4096):
        lib = _lib.load()
        self.shape, self.max_ctx = shape, max_ctx
        cfg = shape.to_c()
        h = ctypes.c_void_p()
        call("mxd_engine_create", ctypes.byref(cfg), max_ctx, ctypes.byref(h))
        self._h = h
        self._lib = lib

    # -- lifecycle ---------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            self._lib.mxd_engine_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- weights -----------------------------------------------------------
    def tensors(self) -> list[tuple[str, int, int]]:
        """(name, device pointer, bytes) of every weight tensor."""
        out = []
        for i in range(self._lib.mxd_engine_num_tensors(self._h)):
            name, ptr, nb, dt = ctypes.c_char_p(), ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_int()
            call("mxd_engine_tensor", self._h, i, ctypes.byref(name), ctypes.byref(ptr), ctypes.byref(nb),
                 ctypes.byref(dt))
            out.append((name.value.decode(), ptr.value, nb.value))
        return out

    def tensor_specs(self) -> list[tuple[str, int, type]]:
        """(name, bytes, numpy dtype) of every weight tensor, in engine order."""
        out = []
        for i in range(self._lib.mxd_engine_num_tensors(self._h)):
            name, ptr, nb, dt = ctypes.c_char_p(), ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_int()
            call("mxd_engine_tensor", self._h, i, ctypes.byref(name), ctypes.byref(ptr), ctypes.byref(nb),
                 ctypes.byref(dt))
            out.append((name.value.decode(), nb.value, np.float16 if dt.value == _lib.MXD_F16 else np.float32))
        return out

    def init_random(self, seed: int, std: float = 0.02, embed_std: float | None = None) -> None:
        """Synthetic weights: every tensor N(0, std^2) from the hash generator,
        the embedding N(0, embed_std^2) if given."""
        call("mxd_engine_init_random", self._h, seed, std)
        if embed_std is not None and embed_std != std:
            self.fill_tensor("embed", seed, embed_std)

    def fill_tensor(self, name: str, seed: int, std: float) -> None:
        idx = self._lib.mxd_engine_find_tensor(self._h, name.encode())
        if idx < 0:
            raise KeyError(name)
        call("mxd_engine_fill_tensor", self._h, idx, seed, std)

    def upload(self, name: str, array: np.ndarray) -> None:
        idx = self._lib.mxd_engine_find_tensor(self._h, name.encode())
        if idx < 0:
            raise KeyError(name)
        a = np.ascontiguousarray(array)
        call("mxd_engine_upload", self._h, idx, a.ctypes.data, a.nbytes)

    def download(self, name: str, dtype) -> np.ndarray:
        """Copy one weight tensor back to the host."""
        idx = self._lib.mxd_engine_find_tensor(self._h, name.encode())
        if idx < 0:
            raise KeyError(name)
        nb = dict((n, b) for n, _, b in self.tensors())[name]
        out = np.empty(nb, np.uint8)
        call("mxd_engine_download", self._h, idx, out.ctypes.data, nb)
        return out.view(dtype)

    # -- tokens ------------------------------------------------------------
    def set_tokens(self, ids: Iterable[int], start: int = 0) -> None:
        a = np.ascontiguousarray(np.asarray(list(ids), dtype=np.int32))
        call("mxd_engine_set_tokens", self._h, a.ctypes.data, start, a.size)

    def tokens(self, start: int, n: int) -> list[int]:
        a = np.empty(n, np.int32)
        call("mxd_engine_get_tokens", self._h, a.ctypes.data, start, n)
        return a.tolist()

    def token(self, at: int) -> int:
        return self.tokens(at, 1)[0]

    def logits(self) -> np.ndarray:
        a = np.empty(self.shape.vocab, np.float32)
        call("mxd_engine_get_logits", self._h, a.ctypes.data)
        return a

    # -- forward passes ------------------------------------------------------
    def step(self, pos: int, sample: bool = True) -> None:
        call("mxd_engine_step", self._h, pos, int(sample))

    def prefill(self, n: int) -> None:
        """Positions 0..n-1 through the decode path; samples tokens[n]. Waits."""
        call("mxd_engine_prefill", self._h, n)
        self.sync()

    def decode(self, pos: int, count: int, wait: bool = True) -> None:
        """Greedy-decode `count` tokens from pos (tokens[pos] must be set)."""
        call("mxd_engine_decode", self._h, pos, count)
        if wait:
            self.sync()

    def sync(self) -> None:
        call("mxd_engine_sync", self._h)

    def generate(self, prompt: list[int], n_new: int) -> list[int]:
        """Prefill the prompt, then n_new - 1 more steps; the n_new greedy tokens."""
        P = len(prompt)
        if P + n_new > self.max_ctx:
            raise ValueError(f"prompt {P} + {n_new} new tokens exceed max_ctx {self.max_ctx}")
        self.set_tokens(prompt)
        self.prefill(P)
        if n_new > 1:
            self.decode(P, n_new - 1)
        return self.tokens(P, n_new)

    def wait_token(self, pos: int) -> int:
        """Wait for the decode step at pos (only) and return its token."""
        tok = ctypes.c_int32()
        call("mxd_engine_wait_token", self._h, pos, ctypes.byref(tok))
        return tok.value

    def decode_streaming(self, pos: int, count: int, emit: Callable[[int], bool], window: int = 3) -> None:
        """Like the reference's decodeStreaming (KL/main.swift:477-491): `window`
        steps stay in flight; the host waits only for the oldest, hands its
        token to emit(token) and queues the next step. emit returning False
        stops generation (steps already queued are drained)."""
        if not 1 <= window <= 16:
            raise ValueError(f"window {window} outside [1, 16] (the engine's ring of step events)")
        queued = done = 0
        stopped = False
        while done < queued or (not stopped and queued < count):
            while not stopped and queued < count and queued - done < window:
                call("mxd_engine_decode", self._h, pos + queued, 1)
                queued += 1
            t = self.wait_token(pos + done)
            done += 1
            if not stopped and not emit(t):
                stopped = True
