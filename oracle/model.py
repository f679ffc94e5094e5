"""The decode step composed from oracle.ops (NumPy; small configurations).

Step order follows the reference's Engine.encodeDecode (KL/main.swift:321-347)
with the Gemma substitutions BASELINE's Gemma-2B shape needs: sqrt(D) embedding
scale (KG/main.swift:397), GeGLU (KG/kernels.metal:205-234), MQA, tied LM head
(KG/main.swift:379-380), (1 + w) RMSNorm weights. Values are rounded to fp32
between ops and K/V to fp16, the storage points of the GPU path.

The Llama-3.2-1B shape of the reference's other engine is covered too: an
untied lm_head (KL/main.swift:306, KL/convert_weights.py:67-68) and Llama-3
RoPE frequency scaling (KL/main.swift:96-107).

Weights are synthetic: hashrng with one tensor id per named tensor (names as
in KL/convert_weights.py:56-69).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import hashrng, ops

F32 = np.float32


@dataclass(frozen=True)
class DecodeConfig:
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 10000.0
    act: str = "gelu_tanh"
    gemma_embed_scale: bool = True   # x = E[tok] * sqrt(D)
    plus_one: bool = True            # RMSNorm weight (1 + w)
    tie_embeddings: bool = True      # LM head = embedding; else a separate lm_head
    # Llama-3 RoPE scaling (factor, low_freq_factor, high_freq_factor,
    # original_max_position_embeddings), or None
    rope_scaling: tuple | None = None

    def inv_freq(self) -> np.ndarray:
        if self.rope_scaling is None:
            return ops.inv_freq(self.head_dim, self.rope_theta)
        return ops.inv_freq_llama3(self.head_dim, self.rope_theta, *self.rope_scaling)

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


GEMMA_2B = DecodeConfig(n_layers=18, dim=2048, n_heads=8, n_kv_heads=1, head_dim=256, ffn_dim=16384, vocab=256000)
TINY = DecodeConfig(n_layers=2, dim=256, n_heads=4, n_kv_heads=1, head_dim=128, ffn_dim=512, vocab=1000)
# The reference's Llama engine model (unsloth/Llama-3.2-1B-Instruct config).
LLAMA32_1B = DecodeConfig(n_layers=16, dim=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn_dim=8192, vocab=128256,
                          eps=1e-5, rope_theta=500000.0, act="silu", gemma_embed_scale=False, plus_one=False,
                          tie_embeddings=True, rope_scaling=(32.0, 1.0, 4.0, 8192))


def tensor_id(name: str) -> int:
    """Tensor id of a named weight for the hash generator."""
    fixed = {"embed": 1, "final_norm": 2, "lm_head": 3}
    if name in fixed:
        return fixed[name]
    layer, kind = name.split(".")
    kinds = ["attn_norm", "wqkv", "wo", "ffn_norm", "wgate", "wup", "wdown"]
    return 1000 + 16 * int(layer[1:]) + kinds.index(kind)


def weight_shapes(cfg: DecodeConfig) -> dict[str, tuple[tuple[int, ...], type]]:
    D, F = cfg.dim, cfg.ffn_dim
    shapes = {"embed": ((cfg.vocab, D), np.float16), "final_norm": ((D,), np.float32)}
    if not cfg.tie_embeddings:
        shapes["lm_head"] = ((cfg.vocab, D), np.float16)
    for l in range(cfg.n_layers):
        shapes[f"l{l}.attn_norm"] = ((D,), np.float32)
        shapes[f"l{l}.wqkv"] = ((cfg.qkv_dim, D), np.float16)
        shapes[f"l{l}.wo"] = ((D, cfg.n_heads * cfg.head_dim), np.float16)
        shapes[f"l{l}.ffn_norm"] = ((D,), np.float32)
        shapes[f"l{l}.wgate"] = ((F, D), np.float16)
        shapes[f"l{l}.wup"] = ((F, D), np.float16)
        shapes[f"l{l}.wdown"] = ((D, F), np.float16)
    return shapes


def make_weights(cfg: DecodeConfig, seed: int, std: float = 0.02, embed_std: float | None = None
                 ) -> dict[str, np.ndarray]:
    """Every tensor N(0, std^2); the embedding N(0, embed_std^2) if given."""
    return {
        name: hashrng.normal(shape, dt, seed, tensor_id(name), embed_std if name == "embed" and embed_std else std)
        for name, (shape, dt) in weight_shapes(cfg).items()
    }


class OracleDecoder:
    """Greedy decoder over a token buffer, mirroring Engine.decode: step(pos) reads
    tokens[pos] and writes argmax to tokens[pos + 1] (KL/main.swift:319-320)."""

    def __init__(self, cfg: DecodeConfig, weights: dict[str, np.ndarray], max_ctx: int, fp16_kv: bool = True):
        self.cfg, self.w, self.max_ctx = cfg, weights, max_ctx
        kv_dt = np.float16 if fp16_kv else np.float64
        self.k = np.zeros((cfg.n_layers, cfg.n_kv_heads, max_ctx, cfg.head_dim), kv_dt)
        self.v = np.zeros((cfg.n_layers, cfg.n_kv_heads, max_ctx, cfg.head_dim), kv_dt)
        self.invf = cfg.inv_freq()
        self.tokens = np.zeros(max_ctx + 1, np.int32)
        self.fp16_kv = fp16_kv

    def _rope_kv(self, l: int, qkv: np.ndarray, pos: int) -> np.ndarray:
        c = self.cfg
        if self.fp16_kv:
            return ops.rope_kv(qkv, self.k[l], self.v[l], self.invf, c.n_heads, c.n_kv_heads, pos)
        hd = c.head_dim
        row = qkv.astype(np.float64)
        q = ops.rope(row[: c.n_heads * hd].reshape(c.n_heads, hd), pos, self.invf)
        k = ops.rope(row[c.n_heads * hd : (c.n_heads + c.n_kv_heads) * hd].reshape(c.n_kv_heads, hd), pos, self.invf)
        self.k[l][:, pos, :] = k
        self.v[l][:, pos, :] = row[(c.n_heads + c.n_kv_heads) * hd :].reshape(c.n_kv_heads, hd)
        return q.reshape(-1)

    def forward(self, pos: int) -> np.ndarray:
        """Logits (fp32) for tokens[pos] at position pos; updates the KV caches."""
        c, w = self.cfg, self.w
        scale = F32(math.sqrt(c.dim)) if c.gemma_embed_scale else F32(1.0)
        x = ops.embed(w["embed"], int(self.tokens[pos]), float(scale)).astype(F32)
        att_scale = float(F32(1.0) / F32(math.sqrt(c.head_dim)))
        for l in range(c.n_layers):
            xn = ops.rmsnorm(x, w[f"l{l}.attn_norm"], c.eps, c.plus_one).astype(F32)
            qkv = ops.matvec(w[f"l{l}.wqkv"], xn).astype(F32)
            q = self._rope_kv(l, qkv, pos).astype(F32)
            att = ops.attention(q, self.k[l], self.v[l], pos + 1, c.n_heads, att_scale).astype(F32)
            x = (x + ops.matvec(w[f"l{l}.wo"], att).astype(F32)).astype(F32)
            xn = ops.rmsnorm(x, w[f"l{l}.ffn_norm"], c.eps, c.plus_one).astype(F32)
            h = ops.gate_up(w[f"l{l}.wgate"], w[f"l{l}.wup"], xn, c.act).astype(F32)
            x = (x + ops.matvec(w[f"l{l}.wdown"], h).astype(F32)).astype(F32)
        xn = ops.rmsnorm(x, w["final_norm"], c.eps, c.plus_one).astype(F32)
        return ops.matvec(self._head(), xn).astype(F32)

    def _head(self) -> np.ndarray:
        """The LM head: the embedding when tied (KG/main.swift:379-380), else
        lm_head (KL/main.swift:306)."""
        return self.w["embed"] if self.cfg.tie_embeddings else self.w["lm_head"]

    def prefill_chunk(self, pos0: int, rows: int, sample: bool = True, half_acts: bool = True) -> np.ndarray | None:
        """The batched prefill of tokens[pos0 .. pos0 + rows) (encodePrefillChunk,
        KL/main.swift:412-446): per layer rmsnorm -> fp16 rows (xnHalf) -> qkv
        product, RoPE + append per position, causal attention (query t over keys
        [0, pos0 + t]), fp16(att) -> wo product added to x, rmsnorm -> fp16 ->
        gate/up, fp16(h) -> down product added to x. With sample, the last row's
        logits (final norm + tied head) are returned and their argmax written to
        tokens[pos0 + rows]. half_acts=False skips the three fp16 roundings (then
        every row equals forward() at its position)."""
        c, w = self.cfg, self.w
        F16 = np.float16 if half_acts else F32
        scale = F32(math.sqrt(c.dim)) if c.gemma_embed_scale else F32(1.0)
        X = np.stack([ops.embed(w["embed"], int(self.tokens[pos0 + t]), float(scale)) for t in range(rows)]).astype(F32)
        att_scale = float(F32(1.0) / F32(math.sqrt(c.head_dim)))
        for l in range(c.n_layers):
            XN = ops.rmsnorm(X, w[f"l{l}.attn_norm"], c.eps, c.plus_one).astype(F32).astype(F16)
            QKV = ops.matvec(w[f"l{l}.wqkv"], XN.T).T.astype(F32)
            Q = np.stack([self._rope_kv(l, QKV[t], pos0 + t) for t in range(rows)]).astype(F32)
            ATT = np.stack([ops.attention(Q[t], self.k[l], self.v[l], pos0 + t + 1, c.n_heads, att_scale)
                            for t in range(rows)]).astype(F32)
            X = (X + ops.matvec(w[f"l{l}.wo"], ATT.astype(F16).T).T.astype(F32)).astype(F32)
            XN = ops.rmsnorm(X, w[f"l{l}.ffn_norm"], c.eps, c.plus_one).astype(F32).astype(F16)
            H = ops.gate_up(w[f"l{l}.wgate"], w[f"l{l}.wup"], XN.T, c.act).T.astype(F32)
            X = (X + ops.matvec(w[f"l{l}.wdown"], H.astype(F16).T).T.astype(F32)).astype(F32)
        if not sample:
            return None
        xn = ops.rmsnorm(X[rows - 1], w["final_norm"], c.eps, c.plus_one).astype(F32)
        logits = ops.matvec(self._head(), xn).astype(F32)
        self.tokens[pos0 + rows] = ops.argmax(logits)
        return logits

    def step(self, pos: int, sample: bool = True) -> tuple[int, float]:
        """One decode step; with sample, tokens[pos + 1] = argmax. Returns (token,
        top-1 minus top-2 logit margin)."""
        logits = self.forward(pos)
        tok = ops.argmax(logits)
        if sample:
            self.tokens[pos + 1] = tok
        top2 = np.partition(logits, -2)[-2:]
        return tok, float(top2[1] - top2[0])

    def generate(self, prompt: list[int], n_new: int, prefill_rows: int | None = None) -> tuple[list[int], list[float]]:
        """Prefill, then n_new - 1 more steps: returns the n_new greedy tokens
        tokens[P .. P + n_new) and their top-2 margins. Prefill is token by token
        through the decode path (the reference's --no-gemm prefill,
        KL/main.swift:367-368) or, with prefill_rows and P > 1, batched in chunks
        of that many rows (prefill(n:useGemm:), KL/main.swift:357-365)."""
        P = len(prompt)
        self.tokens[:P] = prompt
        margins = []
        start = 0
        if prefill_rows and P > 1:
            done = 0
            while done < P:
                rows = min(prefill_rows, P - done)
                lg = self.prefill_chunk(done, rows, sample=done + rows == P)
                done += rows
            top2 = np.partition(lg, -2)[-2:]
            margins.append(float(top2[1] - top2[0]))
            start = P
        for pos in range(start, P + n_new - 1):
            _, m = self.step(pos, sample=pos >= P - 1)
            if pos >= P - 1:
                margins.append(m)
        return [int(t) for t in self.tokens[P : P + n_new]], margins
