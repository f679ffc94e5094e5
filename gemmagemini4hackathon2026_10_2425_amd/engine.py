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


@dataclass(frozen=True)
class Gemma4Layer:
    """Per-layer facts of a Gemma-4 text model (mxd_gemma4_layer), as the
    reference's converter resolves them (KG/convert_weights.py engine_config)."""

    head_dim: int
    ffn_dim: int
    sliding: bool
    kv_layer: int
    rope_pairs: int
    rope_theta: float
    layer_scalar: float = 1.0


@dataclass(frozen=True)
class Gemma4Shape:
    """A Gemma-4 text model (mxd_gemma4_config; KG/main.swift:80-101)."""

    dim: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    ple_dim: int
    ple_vocab: int
    window: int
    layers: tuple
    rms_eps: float = 1e-6
    softcap: float = 30.0

    @property
    def n_layers(self) -> int:
        return len(self.layers)

    def to_c(self) -> tuple[_lib.Gemma4Config, ctypes.Array]:
        """The C config and the layer array it points at (keep both alive)."""
        arr = (_lib.Gemma4Layer * self.n_layers)(*[
            _lib.Gemma4Layer(y.head_dim, y.ffn_dim, int(y.sliding), y.kv_layer, y.rope_pairs, y.rope_theta,
                             y.layer_scalar) for y in self.layers])
        cfg = _lib.Gemma4Config(self.n_layers, self.dim, self.n_heads, self.n_kv_heads, self.vocab, self.ple_dim,
                                self.ple_vocab, self.window, self.rms_eps, self.softcap, arr)
        return cfg, arr

    @property
    def weight_bytes(self) -> int:
        """Bytes of weights one decode step streams: every layer's matrices and
        norms, the per-layer-embedding projection and the tied head; of the
        per-layer-embedding table only the token's row."""
        D, P, L, NH = self.dim, self.ple_dim, self.n_layers, self.n_heads
        b = 2 * self.vocab * D + 2 * L * P * D + 2 * L * P + 4 * (P + D)
        for l, y in enumerate(self.layers):
            own = y.kv_layer == l
            qkv = (NH + (2 * self.n_kv_heads if own else 0)) * y.head_dim
            b += 2 * (qkv * D + D * NH * y.head_dim + 3 * y.ffn_dim * D + 2 * P * D)
            b += 4 * (4 * D + y.head_dim * (2 if own else 1))
        return b

    @staticmethod
    def layers_from_hf(c: dict, layer_scalars=None) -> tuple:
        """Per-layer facts from an HF Gemma-4 text config, as
        KG/convert_weights.py engine_config resolves them: a KV-shared layer
        (index >= n_layers - num_kv_shared_layers) reads the cache of the last
        non-shared layer of its type and, with use_double_wide_mlp, has twice
        the MLP width; "proportional" RoPE rotates partial_rotary_factor of
        the pairs."""
        types = list(c["layer_types"])
        n = int(c["num_hidden_layers"])
        if len(types) != n:
            raise ValueError(f"layer_types has {len(types)} entries for {n} layers")
        first_shared = n - int(c.get("num_kv_shared_layers", 0) or 0)
        last_of_type = {t: i for i, t in enumerate(types[:first_shared])}
        out = []
        for i, t in enumerate(types):
            if t not in ("sliding_attention", "full_attention"):
                raise ValueError(f"layer type {t!r} is not supported")
            sliding = t == "sliding_attention"
            hd = int(c["head_dim"] if sliding else c.get("global_head_dim") or c["head_dim"])
            rope = c["rope_parameters"][t]
            if rope.get("rope_type", "default") == "default":
                pairs = hd // 2
            elif rope["rope_type"] == "proportional":
                pairs = int(rope.get("partial_rotary_factor", 1.0) * hd // 2)
            else:
                raise ValueError(f"rope type {rope['rope_type']!r} is not supported (default or proportional)")
            shared = i >= first_shared
            if shared and t not in last_of_type:
                raise ValueError(f"layer {i} shares the cache of a {t} layer, but none precedes it")
            double = bool(c.get("use_double_wide_mlp", False)) and shared
            out.append(Gemma4Layer(head_dim=hd, ffn_dim=int(c["intermediate_size"]) * (2 if double else 1),
                                   sliding=sliding, kv_layer=last_of_type[t] if shared else i, rope_pairs=pairs,
                                   rope_theta=float(rope["rope_theta"]),
                                   layer_scalar=1.0 if layer_scalars is None else float(layer_scalars[i])))
        return tuple(out)

    @classmethod
    def from_hf(cls, c: dict, layers=None) -> "Gemma4Shape":
        """Shape of an HF Gemma-4 text config (the keys KG/main.swift:86-95
        reads); layers: the resolved per-layer facts, else layers_from_hf(c)."""
        if int(c.get("num_key_value_heads", 1)) < 1:
            raise ValueError("num_key_value_heads must be positive")
        if c.get("enable_moe_block") or c.get("attention_k_eq_v"):
            raise ValueError("only the dense Gemma-4 layout (E2B / E4B) is supported")
        return cls(dim=int(c["hidden_size"]), n_heads=int(c["num_attention_heads"]),
                   n_kv_heads=int(c.get("num_key_value_heads", 1)), vocab=int(c["vocab_size"]),
                   ple_dim=int(c["hidden_size_per_layer_input"]),
                   ple_vocab=int(c.get("vocab_size_per_layer_input", c["vocab_size"])),
                   window=int(c["sliding_window"]), layers=tuple(layers) if layers else cls.layers_from_hf(c),
                   rms_eps=float(c.get("rms_norm_eps", 1e-6)),
                   softcap=float(c.get("final_logit_softcapping") or 0.0))


# google/gemma-4-E2B-it's text model (KG/PLAN.md, "The model"): 35 layers of
# [sliding x4, full] x7, hidden 1536, 8 query heads / 1 KV head, head_dim 256
# (sliding, window 512, RoPE theta 1e4) / 512 (full, theta 1e6, a quarter of
# the pairs rotated), the last 20 layers sharing the caches of layers 13 / 14
# with double-width MLPs (6144 -> 12288), per-layer embeddings of 256, vocab
# 262144, softcap 30. Layer scalars are learned (1 here: synthetic weights).
GEMMA4_E2B_TEXT_CONFIG = {
    "hidden_size": 1536, "num_hidden_layers": 35, "num_attention_heads": 8, "num_key_value_heads": 1,
    "head_dim": 256, "global_head_dim": 512, "intermediate_size": 6144, "vocab_size": 262144,
    "vocab_size_per_layer_input": 262144, "hidden_size_per_layer_input": 256, "sliding_window": 512,
    "rms_norm_eps": 1e-6, "final_logit_softcapping": 30.0, "num_kv_shared_layers": 20, "use_double_wide_mlp": True,
    "layer_types": (["sliding_attention"] * 4 + ["full_attention"]) * 7,
    "rope_parameters": {"sliding_attention": {"rope_type": "default", "rope_theta": 10000.0},
                        "full_attention": {"rope_type": "proportional", "partial_rotary_factor": 0.25,
                                           "rope_theta": 1000000.0}},
}
GEMMA4_E2B = Gemma4Shape.from_hf(GEMMA4_E2B_TEXT_CONFIG)


class Engine:
    """Device-resident greedy decoder. Token t of a run is written by the GPU
    into tokens[t + 1]; decode() queues all steps without a host sync. The
    shape picks the model family: ModelShape (Llama / Gemma) or Gemma4Shape."""

    def __init__(self, shape: ModelShape | Gemma4Shape, max_ctx: int = 4096):
        lib = _lib.load()
        self.shape, self.max_ctx = shape, max_ctx
        h = ctypes.c_void_p()
        if isinstance(shape, Gemma4Shape):
            cfg, _layers = shape.to_c()
            call("mxd_engine_create_gemma4", ctypes.byref(cfg), max_ctx, ctypes.byref(h))
        else:
            cfg = shape.to_c()
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
        """fp32 logits of the last sampled step (Gemma-4: after the softcap)."""
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
