"""Write tests/golden/hf_gemma4_tiny.npz: logits and greedy tokens of transformers'
Gemma4ForCausalLM (float64) on a tiny Gemma-4-shaped text config carrying every
feature of the reference's Gemma-4 engine (ios_kernels/kernels/
google__gemma-4-E2B-it/kernel_metal_f16_20261025-1225/): sliding and full
attention layers with head_dim 64 / 128, a sliding window of 16, proportional
RoPE (a quarter of the pairs rotated) on full layers, two KV-shared layers with
double-width MLPs, q/k/v norms, sandwich norms, per-layer embeddings (dim 32),
per-layer scalars and the final logit softcap.

    python tests/golden/make_hf_gemma4_golden.py

Runs in the build container only (locally installed transformers; nothing is
downloaded). Weights are the oracle's synthetic tensors (oracle/gemma4.py, the
q/k norm weights scaled by QK_NORM_SCALE),
loaded by the names of the reference's converter (KG/convert_weights.py):
wqkv splits into q/k/v_proj rows, the layer scalars come from the config.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import gemma4 as g4  # noqa: E402

OUT = Path(__file__).resolve().parent / "hf_gemma4_tiny.npz"
SEED = 36
# q_norm / k_norm weights x 0.25: softer attention, so the fp16 K/V of the
# device path moves the logits by < 1e-3 and the greedy margins stay > 2% of
# the largest logit (checked when the fixture was made).
QK_NORM_SCALE = 0.25
PROMPT = [5, 17, 999, 3, 250, 250, 42, 7, 100, 311, 12, 600, 31, 2, 77, 5, 444, 9, 8, 123]
N_NEW = 12


def hf_model(cfg: g4.G4Config, w: dict):
    from transformers import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM

    types = ["sliding_attention" if lay.sliding else "full_attention" for lay in cfg.layers]
    sl = next(lay for lay in cfg.layers if lay.sliding)
    fl = next(lay for lay in cfg.layers if not lay.sliding)
    n_shared = sum(1 for l, lay in enumerate(cfg.layers) if lay.kv_layer != l)
    hc = Gemma4TextConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.dim, intermediate_size=cfg.layers[0].ffn_dim,
        num_hidden_layers=cfg.n_layers, num_attention_heads=cfg.n_heads, num_key_value_heads=1,
        head_dim=sl.head_dim, global_head_dim=fl.head_dim, hidden_activation="gelu_pytorch_tanh",
        max_position_embeddings=256, rms_norm_eps=cfg.eps, tie_word_embeddings=True, sliding_window=cfg.window,
        layer_types=types, final_logit_softcapping=cfg.softcap, vocab_size_per_layer_input=cfg.ple_vocab,
        hidden_size_per_layer_input=cfg.ple_dim, num_kv_shared_layers=n_shared, use_double_wide_mlp=True,
        pad_token_id=0, bos_token_id=2, eos_token_id=1,
        rope_parameters={"sliding_attention": {"rope_type": "default", "rope_theta": sl.rope_theta},
                         "full_attention": {"rope_type": "proportional",
                                            "partial_rotary_factor": 2 * fl.rope_pairs / fl.head_dim,
                                            "rope_theta": fl.rope_theta}})
    hc._attn_implementation = "eager"
    model = Gemma4ForCausalLM(hc).to(torch.float64).eval()
    m = "model."
    sd = {m + "embed_tokens.weight": w["embed"], m + "embed_tokens_per_layer.weight": w["ple_embed"],
          m + "per_layer_model_projection.weight": w["ple_proj"], m + "per_layer_projection_norm.weight": w["ple_norm"],
          m + "norm.weight": w["final_norm"]}
    for l, lay in enumerate(cfg.layers):
        p = f"{m}layers.{l}."
        hd, q = lay.head_dim, cfg.n_heads * lay.head_dim
        qkv = w[f"l{l}.wqkv"]
        sd[p + "self_attn.q_proj.weight"] = qkv[:q]
        sd[p + "self_attn.q_norm.weight"] = w[f"l{l}.q_norm"]
        if lay.kv_layer == l:
            sd[p + "self_attn.k_proj.weight"] = qkv[q : q + hd]
            sd[p + "self_attn.v_proj.weight"] = qkv[q + hd :]
            sd[p + "self_attn.k_norm.weight"] = w[f"l{l}.k_norm"]
        sd[p + "self_attn.o_proj.weight"] = w[f"l{l}.wo"]
        sd[p + "input_layernorm.weight"] = w[f"l{l}.attn_norm"]
        sd[p + "post_attention_layernorm.weight"] = w[f"l{l}.post_attn_norm"]
        sd[p + "pre_feedforward_layernorm.weight"] = w[f"l{l}.ffn_norm"]
        sd[p + "post_feedforward_layernorm.weight"] = w[f"l{l}.post_ffn_norm"]
        sd[p + "mlp.gate_proj.weight"] = w[f"l{l}.wgate"]
        sd[p + "mlp.up_proj.weight"] = w[f"l{l}.wup"]
        sd[p + "mlp.down_proj.weight"] = w[f"l{l}.wdown"]
        sd[p + "per_layer_input_gate.weight"] = w[f"l{l}.ple_gate"]
        sd[p + "per_layer_projection.weight"] = w[f"l{l}.ple_out"]
        sd[p + "post_per_layer_input_norm.weight"] = w[f"l{l}.post_ple_norm"]
        sd[p + "layer_scalar"] = np.array([lay.layer_scalar])
    state = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(state, strict=False)
    missing = [k for k in missing if k != "lm_head.weight"]
    assert not missing and not unexpected, (missing, unexpected)
    return model


def main() -> None:
    cfg = g4.G4_TINY
    model = hf_model(cfg, g4.make_weights(cfg, SEED, qk_norm_scale=QK_NORM_SCALE))
    with torch.no_grad():
        logits = model(torch.tensor([PROMPT])).logits[0].numpy()
        gen = model.generate(torch.tensor([PROMPT]), max_new_tokens=N_NEW, do_sample=False, temperature=None,
                             top_p=None, top_k=None)[0, len(PROMPT):].tolist()
    np.savez_compressed(OUT, seed=SEED, qk_norm_scale=QK_NORM_SCALE, prompt=np.array(PROMPT, np.int32),
                        logits=logits.astype(np.float64), greedy=np.array(gen, np.int32))
    print(f"wrote {OUT}: logits {logits.shape}, greedy {gen}")


if __name__ == "__main__":
    main()
