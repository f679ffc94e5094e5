"""The Gemma-4 decode step composed from oracle.ops (NumPy; small configurations).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference's Gemma-4 engine (KG = ios_kernels/kernels/
google__gemma-4-E2B-it/kernel_metal_f16_20261025-1225/): the decode order of
encodeDecode (KG/main.swift:394-423), the per-layer facts its converter
resolves (KG/convert_weights.py engine_config: head_dim 256 sliding / 512
full, ffn_dim doubled on KV-shared layers, kv_layer, rope theta and rotated
pairs, layer_scalar), and the operators:
  rmsnorm_add      x = (x + rmsnorm(src) * w) * post          KG/kernels.metal:106-125
  ple_combine      ple = (rmsnorm(proj * D^-0.5) * w + ple) / sqrt(2)   :132-149
  qkv_norm_rope    per-head RMSNorm of q, k (weights) and v (none), RoPE on
                   the first rope_pairs pairs, k, v to the cache     :246-304
  attention        scale 1, sliding layers over keys (pos - window, pos]
                                                                     :306-393
  LM head          tied embedding; logits 30 tanh(logits / 30) only where
                   they are dumped (KG/main.swift:657-662), argmax unchanged
RMSNorm multiplies by w (not 1 + w); the embedding is scaled by sqrt(D), the
per-layer table by sqrt(P). Values are rounded to fp32 between ops and K/V to
fp16, the storage points of the GPU path. Pinned against transformers'
Gemma4ForCausalLM on a tiny config (tests/golden/hf_gemma4_tiny.npz).

Synthetic weights: hashrng N(0, std^2) per named tensor; norm weights are
1 + N(0, std^2) (the fp32 sum), so activations keep their scale.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import hashrng, ops

F16, F32, F64 = np.float16, np.float32, np.float64


@dataclass(frozen=True)
class G4Layer:
    head_dim: int
    ffn_dim: int
    sliding: bool
    kv_layer: int
    rope_theta: float
    rope_pairs: int
    layer_scalar: float = 1.0


@dataclass(frozen=True)
class G4Config:
    dim: int
    n_heads: int
    vocab: int
    ple_dim: int
    ple_vocab: int
    window: int
    layers: tuple = field(default_factory=tuple)
    eps: float = 1e-6
    softcap: float = 30.0

    @property
    def n_layers(self) -> int:
        return len(self.layers)

    def inv_freq(self, l: int) -> np.ndarray:
        """theta^(-2i/hd) for the first rope_pairs pairs, 0 (no rotation) after
        (KG/main.swift:97-99: default RoPE on sliding layers, "proportional"
        on full ones)."""
        lay = self.layers[l]
        i = np.arange(lay.head_dim // 2, dtype=F64)
        f = 1.0 / lay.rope_theta ** (2.0 * i / lay.head_dim)
        return np.where(i < lay.rope_pairs, f, 0.0).astype(F32)


def layers_from_types(types: list[str], head_dim: int, global_head_dim: int, ffn_dim: int, n_shared: int,
                      double_wide: bool, sliding_theta: float = 1e4, full_theta: float = 1e6,
                      full_partial: float = 0.25, scalars=None) -> tuple:
    """Per-layer facts from the HF text config, as the reference's converter
    resolves them (KG/convert_weights.py engine_config): a KV-shared layer
    (index >= n_layers - n_shared) reads the cache of the last non-shared
    layer of its type and has a double-width MLP when configured."""
    n = len(types)
    first_shared = n - n_shared
    last_of_type = {t: i for i, t in enumerate(types[:first_shared])}
    out = []
    for i, t in enumerate(types):
        sliding = t == "sliding_attention"
        hd = head_dim if sliding else global_head_dim
        pairs = hd // 2 if sliding else int(full_partial * hd // 2)
        shared = i >= first_shared
        out.append(G4Layer(head_dim=hd, ffn_dim=ffn_dim * (2 if double_wide and shared else 1), sliding=sliding,
                           kv_layer=last_of_type[t] if shared else i,
                           rope_theta=sliding_theta if sliding else full_theta, rope_pairs=pairs,
                           layer_scalar=1.0 if scalars is None else float(scalars[i])))
    return tuple(out)


G4_TINY_TYPES = ["sliding_attention", "sliding_attention", "full_attention", "sliding_attention",
                 "sliding_attention", "full_attention"]
G4_TINY = G4Config(dim=256, n_heads=4, vocab=1000, ple_dim=32, ple_vocab=1000, window=16,
                   layers=layers_from_types(G4_TINY_TYPES, 64, 128, 512, n_shared=2, double_wide=True,
                                            scalars=[0.9, 1.1, 0.8, 1.0, 1.2, 0.7]))
# google/gemma-4-E2B text model: 35 layers [sliding x4, full] x7, hidden 1536,
# 8 Q heads / 1 KV head, head_dim 256 / 512, window 512, 20 KV-shared layers
# with double-width MLPs, PLE dim 256 (KG/PLAN.md:25-44).
G4_E2B = G4Config(dim=1536, n_heads=8, vocab=262144, ple_dim=256, ple_vocab=262144, window=512,
                  layers=layers_from_types((["sliding_attention"] * 4 + ["full_attention"]) * 7, 256, 512, 6144,
                                           n_shared=20, double_wide=True))

LAYER_KINDS = ["attn_norm", "wqkv", "wo", "ffn_norm", "wgate", "wup", "wdown", "q_norm", "k_norm", "post_attn_norm",
               "post_ffn_norm", "ple_gate", "ple_out", "post_ple_norm"]
NORMS = {"attn_norm", "ffn_norm", "q_norm", "k_norm", "post_attn_norm", "post_ffn_norm", "post_ple_norm",
         "final_norm", "ple_norm"}


def tensor_id(name: str) -> int:
    """Tensor id of a named weight for the hash generator: embed 1, final_norm 2,
    ple_embed 4, ple_proj 5, ple_norm 6, layer l: 1000 + 16 l + kind index."""
    fixed = {"embed": 1, "final_norm": 2, "ple_embed": 4, "ple_proj": 5, "ple_norm": 6}
    if name in fixed:
        return fixed[name]
    layer, kind = name.split(".")
    return 1000 + 16 * int(layer[1:]) + LAYER_KINDS.index(kind)


def weight_shapes(cfg: G4Config) -> dict[str, tuple[tuple[int, ...], type]]:
    """Tensor names and shapes of the reference's converted file
    (KG/convert_weights.py: wqkv is q|k|v, q only on KV-shared layers; a
    KV-shared layer has no k_norm)."""
    D, P, L = cfg.dim, cfg.ple_dim, cfg.n_layers
    s = {"embed": ((cfg.vocab, D), F16), "ple_embed": ((cfg.ple_vocab, L * P), F16), "ple_proj": ((L * P, D), F16),
         "ple_norm": ((P,), F32)}
    for l, lay in enumerate(cfg.layers):
        hd, own = lay.head_dim, lay.kv_layer == l
        q = cfg.n_heads * hd
        s[f"l{l}.attn_norm"] = ((D,), F32)
        s[f"l{l}.wqkv"] = ((q + 2 * hd if own else q, D), F16)
        s[f"l{l}.q_norm"] = ((hd,), F32)
        if own:
            s[f"l{l}.k_norm"] = ((hd,), F32)
        s[f"l{l}.wo"] = ((D, q), F16)
        s[f"l{l}.post_attn_norm"] = ((D,), F32)
        s[f"l{l}.ffn_norm"] = ((D,), F32)
        s[f"l{l}.wgate"] = ((lay.ffn_dim, D), F16)
        s[f"l{l}.wup"] = ((lay.ffn_dim, D), F16)
        s[f"l{l}.wdown"] = ((D, lay.ffn_dim), F16)
        s[f"l{l}.post_ffn_norm"] = ((D,), F32)
        s[f"l{l}.ple_gate"] = ((P, D), F16)
        s[f"l{l}.ple_out"] = ((D, P), F16)
        s[f"l{l}.post_ple_norm"] = ((D,), F32)
    s["final_norm"] = ((D,), F32)
    return s


def make_weights(cfg: G4Config, seed: int, std: float = 0.02, qk_norm_scale: float = 1.0) -> dict[str, np.ndarray]:
    """qk_norm_scale multiplies the q_norm / k_norm weights (an fp32 product):
    below 1 it softens the attention (scale 1 over unit-RMS q and k), which
    keeps small test models well conditioned under fp16 K/V."""
    w = {}
    for name, (shape, dt) in weight_shapes(cfg).items():
        v = hashrng.normal(shape, dt, seed, tensor_id(name), std)
        kind = name.split(".")[-1]
        w[name] = (v + F32(1.0)).astype(F32) if kind in NORMS else v
        if kind in ("q_norm", "k_norm") and qk_norm_scale != 1.0:
            w[name] = (w[name] * F32(qk_norm_scale)).astype(F32)
    return w


def _h(v, half: bool):
    """v rounded to fp16 (and back to fp32) when half, else unchanged."""
    return np.asarray(v).astype(F16).astype(F32) if half else v


def rmsnorm_w(x, w, eps):
    """x * rsqrt(mean(x^2) + eps) * w (w None: no weight), fp64."""
    x = np.asarray(x, dtype=F64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return y if w is None else y * np.asarray(w, dtype=F64)


class G4Decoder:
    """Greedy decoder over a token buffer: step(pos) reads tokens[pos] and, with
    sample, writes argmax to tokens[pos + 1] (KG/main.swift:394-423)."""

    def __init__(self, cfg: G4Config, weights: dict[str, np.ndarray], max_ctx: int, fp16_kv: bool = True):
        """fp16_kv=False keeps K/V unrounded in fp64 (for the comparison with
        transformers in float64)."""
        self.cfg, self.w, self.max_ctx = cfg, weights, max_ctx
        kv = F16 if fp16_kv else F64
        self.k = {l: np.zeros((max_ctx, lay.head_dim), kv) for l, lay in enumerate(cfg.layers) if lay.kv_layer == l}
        self.v = {l: np.zeros((max_ctx, lay.head_dim), kv) for l, lay in enumerate(cfg.layers) if lay.kv_layer == l}
        self.invf = [cfg.inv_freq(l) for l in range(cfg.n_layers)]
        self.tokens = np.zeros(max_ctx + 1, np.int32)

    def ple(self, tok: int, x: np.ndarray, half_acts: bool = False) -> np.ndarray:
        """Per-layer inputs [L, P] of a token (KG/main.swift:398-401, ple_combine
        KG/kernels.metal:132-149)."""
        c, w = self.cfg, self.w
        L, P = c.n_layers, c.ple_dim
        tok_part = (w["ple_embed"][tok].astype(F64) * F32(math.sqrt(P))).astype(F32).reshape(L, P)
        proj = ops.matvec(w["ple_proj"], _h(x, half_acts)).astype(F32).reshape(L, P)
        normed = rmsnorm_w(proj.astype(F64) * F32(c.dim ** -0.5), w["ple_norm"], c.eps)
        return ((normed + tok_part.astype(F64)) * (2.0 ** -0.5)).astype(F32)

    def forward(self, pos: int, half_acts: bool = False) -> np.ndarray:
        """Logits (fp32, before the softcap) for tokens[pos] at position pos.
        half_acts: the activations that enter a product are rounded to fp16
        first, as the reference's batched prefill chunk stores them
        (xnHalf / attHalf / hidHalf / plegHalf, KG/main.swift:486-520)."""
        c, w = self.cfg, self.w
        D, NH = c.dim, c.n_heads
        tok = int(self.tokens[pos])
        x = ops.embed(w["embed"], tok, float(F32(math.sqrt(D)))).astype(F32)
        ple = self.ple(tok, x, half_acts)
        for l, lay in enumerate(c.layers):
            hd, own = lay.head_dim, lay.kv_layer == l
            xn = _h(rmsnorm_w(x, w[f"l{l}.attn_norm"], c.eps).astype(F32), half_acts)
            qkv = ops.matvec(w[f"l{l}.wqkv"], xn).astype(F32)
            q = rmsnorm_w(qkv[: NH * hd].reshape(NH, hd), w[f"l{l}.q_norm"], c.eps).astype(F32)
            q = ops.rope(q, pos, self.invf[l]).astype(F32)
            if own:
                k = rmsnorm_w(qkv[NH * hd : (NH + 1) * hd], w[f"l{l}.k_norm"], c.eps).astype(F32)
                self.k[l][pos] = ops.rope(k, pos, self.invf[l]).astype(F32)
                self.v[l][pos] = rmsnorm_w(qkv[(NH + 1) * hd :], None, c.eps).astype(F32)
            start = max(0, pos - c.window + 1) if lay.sliding else 0
            kc, vc = self.k[lay.kv_layer], self.v[lay.kv_layer]
            att = ops.attention(q.reshape(-1), kc[None, start : pos + 1], vc[None, start : pos + 1], pos + 1 - start,
                                NH, 1.0).astype(F32)
            a = ops.matvec(w[f"l{l}.wo"], _h(att, half_acts))
            x = (x.astype(F64) + rmsnorm_w(a.astype(F32), w[f"l{l}.post_attn_norm"], c.eps)).astype(F32)
            xn = _h(rmsnorm_w(x, w[f"l{l}.ffn_norm"], c.eps).astype(F32), half_acts)
            h = ops.gate_up(w[f"l{l}.wgate"], w[f"l{l}.wup"], xn, "gelu_tanh").astype(F32)
            m = ops.matvec(w[f"l{l}.wdown"], _h(h, half_acts))
            x = (x.astype(F64) + rmsnorm_w(m.astype(F32), w[f"l{l}.post_ffn_norm"], c.eps)).astype(F32)
            gi = ops.matvec(w[f"l{l}.ple_gate"], _h(x, half_acts)).astype(F32)
            g = _h((ops.gelu_tanh(gi) * ple[l]).astype(F32), half_acts)
            p = ops.matvec(w[f"l{l}.ple_out"], g)
            x = ((x.astype(F64) + rmsnorm_w(p.astype(F32), w[f"l{l}.post_ple_norm"], c.eps)) * lay.layer_scalar
                 ).astype(F32)
        xn = rmsnorm_w(x, w["final_norm"], c.eps).astype(F32)
        return ops.matvec(w["embed"], xn).astype(F32)

    def softcap(self, logits: np.ndarray) -> np.ndarray:
        cap = self.cfg.softcap
        return (cap * np.tanh(np.asarray(logits, F64) / cap)).astype(F32) if cap else logits

    def step(self, pos: int, sample: bool = True) -> tuple[int, float]:
        logits = self.forward(pos)
        tok = ops.argmax(logits)
        if sample:
            self.tokens[pos + 1] = tok
        top2 = np.partition(logits, -2)[-2:]
        return tok, float(top2[1] - top2[0])

    def generate(self, prompt: list[int], n_new: int) -> tuple[list[int], list[float]]:
        P = len(prompt)
        self.tokens[:P] = prompt
        margins = []
        for pos in range(P + n_new - 1):
            _, m = self.step(pos, sample=pos >= P - 1)
            if pos >= P - 1:
                margins.append(m)
        return [int(t) for t in self.tokens[P : P + n_new]], margins
