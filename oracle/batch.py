"""Ragged-batch decode of one transformer layer, composed from oracle.ops.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

B sequences decode one token each; sequence b has seq_lens[b] - 1 cached
positions before the step and appends its new token at position
seq_lens[b] - 1. The layer is Llama-shaped (plain-w RMSNorm, SwiGLU, GQA)
with int8 block-32 weights, the shape of the batched decode the library runs
on a paged KV cache. The step order is the reference's per-layer order
(KL/main.swift:321-347): rmsnorm -> qkv -> rope_kv -> attention -> o (+x) ->
rmsnorm -> gate/up -> down (+x). Values are rounded where the GPU path stores
them: the normed activations, the attention output and the GLU output to fp16
(the fp16 operands of the batched matrix products, f32_to_f16 at
KL/kernels.metal:361-365), the projections and the residual to fp32, K/V to
the caches' dtype (fp16 as on the device). Caches here are per sequence in the
reference's layout [n_kv, ctx, hd].

Pins (tests/test_oracle.py): dequant by closed forms (its fp16 mode within
half an fp16 ulp of each exact weight, and equal to numpy's own fp16
rounding of it); gemm_q8b32 row by row
against ops.matvec_q8b32 and against math.fsum brute force; gate_up_rows row
by row against ops.gate_up_q8b32; layer_step on a ragged, staggered batch
against each sequence stepped alone, and, without the fp16 activation
roundings and with fp64 caches, against transformers' LlamaDecoderLayer in
float64 (tests/golden/hf_llama_layer.npz).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import hashrng, ops

F16, F32, F64 = np.float16, np.float32, np.float64


@dataclass(frozen=True)
class LayerConfig:
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    eps: float = 1e-5
    rope_theta: float = 10000.0
    act: str = "silu"
    plus_one: bool = False

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


LLAMA3_8B_LAYER = LayerConfig(dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=14336)

MATRICES = ("wqkv", "wo", "wgate", "wup", "wdown")


def synthetic_layer(cfg: LayerConfig, seed: int, std: float = 0.02) -> dict:
    """int8 block-32 weights quantised (ops.quantize_q8b32) from hash-generator
    N(0, std^2) fp16 draws, and fp32 norm weights 1 + N(0, std^2); tensor ids
    1000 + {wqkv 1, wo 2, wgate 4, wup 5, wdown 6, attn_norm 0, ffn_norm 3}."""
    D, F, QD = cfg.dim, cfg.ffn_dim, cfg.n_heads * cfg.head_dim
    dims = {"wqkv": (cfg.qkv_dim, D, 1), "wo": (D, QD, 2), "wgate": (F, D, 4), "wup": (F, D, 5),
            "wdown": (D, F, 6)}
    W = {name: ops.quantize_q8b32(hashrng.normal((M, K), F16, seed, 1000 + tid, std))
         for name, (M, K, tid) in dims.items()}
    for name, tid in (("attn_norm", 0), ("ffn_norm", 3)):
        W[name] = (1.0 + hashrng.normal((D,), F32, seed, 1000 + tid, std).astype(F64)).astype(F32)
    return W


def dequant(q: np.ndarray, s: np.ndarray, f16: bool = False) -> np.ndarray:
    """fp64 weights q * s (exact: an fp16 scale times an int8 fits in fp64);
    f16: each product rounded to fp16 (nearest even), the weights the batched
    matrix-core products feed their fp16 MFMAs."""
    M, K = q.shape
    w = (q.reshape(M, K // 32, 32).astype(F64) * s.astype(F64)[:, :, None]).reshape(M, K)
    return w.astype(F16).astype(F64) if f16 else w


def gemm_q8b32(q: np.ndarray, s: np.ndarray, X: np.ndarray, f16_weights: bool = False) -> np.ndarray:
    """Y[b] = matvec_q8b32(q, s, X[b]) for every row b, in fp64 (one
    dequantisation, one BLAS product); f16_weights: with the dequantised
    weights rounded to fp16 (the matrix-core path, from 16 rows)."""
    return np.asarray(X, dtype=F64) @ dequant(q, s, f16_weights).T


def gate_up_rows(qg, sg, qu, su, X, act: str, f16_weights: bool = False) -> np.ndarray:
    g, u = gemm_q8b32(qg, sg, X, f16_weights), gemm_q8b32(qu, su, X, f16_weights)
    return (ops.gelu_tanh(g) if act == "gelu_tanh" else ops.silu(g)) * u


def layer_step(cfg: LayerConfig, W: dict, X: np.ndarray, kcaches: list, vcaches: list,
               seq_lens: np.ndarray, half_acts: bool = True, f16_weights: bool = False) -> np.ndarray:
    """One decode step of the layer for every sequence; returns the new residual
    rows (fp32 [B, D]) and appends each sequence's k, v to its caches (rounded
    to the caches' dtype).

    W: attn_norm, ffn_norm (fp32 [D]); wqkv, wo, wgate, wup, wdown as (q int8,
    s fp16) pairs. kcaches[b], vcaches[b]: [n_kv, ctx_b, hd], ctx_b >=
    seq_lens[b]. half_acts=False skips the three fp16 roundings of the
    products' activation operands (then, with fp64 caches, the step is the
    layer's exact arithmetic up to the fp32 storage of its outputs);
    f16_weights rounds the dequantised weights to fp16 (the matrix-core
    products of a batch of at least 16 rows)."""
    B = X.shape[0]
    NH, NKV, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    H = F16 if half_acts else F32
    invf = ops.inv_freq(hd, cfg.rope_theta)
    scale = 1.0 / math.sqrt(hd)
    X = np.asarray(X, dtype=F32)
    xn = ops.rmsnorm(X, W["attn_norm"], cfg.eps, cfg.plus_one).astype(H)
    fw = f16_weights
    qkv = gemm_q8b32(*W["wqkv"], xn, fw).astype(F32)
    att = np.empty((B, NH * hd), dtype=F32)
    for b in range(B):
        pos = int(seq_lens[b]) - 1
        q = ops.rope_kv(qkv[b], kcaches[b], vcaches[b], invf, NH, NKV, pos).astype(F32)
        att[b] = ops.attention(q, kcaches[b], vcaches[b], pos + 1, NH, scale)
    x1 = (X.astype(F64) + gemm_q8b32(*W["wo"], att.astype(H), fw)).astype(F32)
    xn2 = ops.rmsnorm(x1, W["ffn_norm"], cfg.eps, cfg.plus_one).astype(H)
    h = gate_up_rows(*W["wgate"], *W["wup"], xn2, cfg.act, fw).astype(F32).astype(H)
    return (x1.astype(F64) + gemm_q8b32(*W["wdown"], h, fw)).astype(F32)
