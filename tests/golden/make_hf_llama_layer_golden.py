"""Write tests/golden/hf_llama_layer.npz: outputs of transformers'
LlamaDecoderLayer (float64) for a tiny Llama-shaped layer whose weights are
the oracle's synthetic int8 block-32 weights, dequantised. It pins
oracle.batch.layer_step (the checker of the ragged-batch path): layer order,
GQA head mapping, SwiGLU, RoPE at each sequence's own positions and the
residual adds.

    python tests/golden/make_hf_llama_layer_golden.py

Runs in the build container only (it needs the locally installed
transformers; nothing is downloaded). Each sequence b runs through the layer
alone as one causal forward over its LENS[b] input rows (hash-generator
N(0, 1) values, tensor id 500 + b); the test steps the same rows through the
oracle token by token in a staggered ragged batch and compares every row.
RoPE's cos/sin come from the oracle's inv_freq with the angle
fp32(pos) * inv_freq in fp32, as on the device (the inverse frequencies have
their own pins), and are handed to the layer as position_embeddings.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import batch as ob, hashrng, ops  # noqa: E402

OUT = Path(__file__).resolve().parent / "hf_llama_layer.npz"
SEED = 29
CFG = ob.LayerConfig(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, eps=1e-5, rope_theta=500000.0)
LENS = (7, 12, 4)
STARTS = (0, 3, 6)


def inputs(b: int) -> np.ndarray:
    return hashrng.normal((LENS[b], CFG.dim), np.float32, SEED, 500 + b, 1.0)


def main() -> None:
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer

    c = CFG
    hc = LlamaConfig(hidden_size=c.dim, intermediate_size=c.ffn_dim, num_attention_heads=c.n_heads,
                     num_key_value_heads=c.n_kv_heads, head_dim=c.head_dim, rms_norm_eps=c.eps,
                     hidden_act="silu", attention_bias=False, mlp_bias=False, num_hidden_layers=1,
                     rope_theta=c.rope_theta, max_position_embeddings=64)
    hc._attn_implementation = "eager"
    layer = LlamaDecoderLayer(hc, layer_idx=0).to(torch.float64).eval()
    W = ob.synthetic_layer(c, SEED)
    nh, nkv, hd = c.n_heads, c.n_kv_heads, c.head_dim
    wqkv = ob.dequant(*W["wqkv"])
    sd = {
        "self_attn.q_proj.weight": wqkv[: nh * hd],
        "self_attn.k_proj.weight": wqkv[nh * hd : (nh + nkv) * hd],
        "self_attn.v_proj.weight": wqkv[(nh + nkv) * hd :],
        "self_attn.o_proj.weight": ob.dequant(*W["wo"]),
        "mlp.gate_proj.weight": ob.dequant(*W["wgate"]),
        "mlp.up_proj.weight": ob.dequant(*W["wup"]),
        "mlp.down_proj.weight": ob.dequant(*W["wdown"]),
        "input_layernorm.weight": W["attn_norm"],
        "post_attention_layernorm.weight": W["ffn_norm"],
    }
    state = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in sd.items()}
    missing, unexpected = layer.load_state_dict(state, strict=True)
    assert not missing and not unexpected, (missing, unexpected)
    invf = ops.inv_freq(hd, c.rope_theta)
    outs = []
    with torch.no_grad():
        for b, n in enumerate(LENS):
            ang = (np.arange(n, dtype=np.float32)[:, None] * invf[None, :]).astype(np.float64)
            emb = np.concatenate([ang, ang], axis=1)
            cos = torch.from_numpy(np.cos(emb))[None]
            sin = torch.from_numpy(np.sin(emb))[None]
            mask = torch.full((n, n), float("-inf"), dtype=torch.float64).triu(1)[None, None]
            x = torch.from_numpy(inputs(b).astype(np.float64))[None]
            y = layer(x, attention_mask=mask, position_ids=torch.arange(n)[None], position_embeddings=(cos, sin))
            y = y[0] if isinstance(y, tuple) else y
            outs.append(y[0].numpy())
    np.savez_compressed(OUT, seed=SEED, lens=np.array(LENS), starts=np.array(STARTS),
                        dims=np.array([c.dim, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim]),
                        eps=c.eps, rope_theta=c.rope_theta, out=np.concatenate(outs).astype(np.float64))
    print(f"wrote {OUT}: {sum(LENS)} rows")


if __name__ == "__main__":
    main()
