"""The tiny Gemma-4 config in transformers' terms, and the oracle's synthetic
weights under transformers' tensor names (Gemma4ForCausalLM: prefix "model.";
the multimodal checkpoint nests the same names under "model.language_model."),
for the HF golden fixture and the converter tests."""

from __future__ import annotations

import numpy as np

from oracle import gemma4 as g4


def text_config(cfg: g4.G4Config) -> dict:
    """An HF Gemma-4 text config (model_type gemma4_text) of a G4Config whose
    sliding / full layers share head_dim / theta / rotated fraction and whose
    KV-shared layers are the last ones (as in every Gemma-4 text model)."""
    sl = next(lay for lay in cfg.layers if lay.sliding)
    fl = next(lay for lay in cfg.layers if not lay.sliding)
    n_shared = sum(1 for l, lay in enumerate(cfg.layers) if lay.kv_layer != l)
    return {
        "model_type": "gemma4_text", "vocab_size": cfg.vocab, "hidden_size": cfg.dim,
        "intermediate_size": cfg.layers[0].ffn_dim, "num_hidden_layers": cfg.n_layers,
        "num_attention_heads": cfg.n_heads, "num_key_value_heads": 1, "head_dim": sl.head_dim,
        "global_head_dim": fl.head_dim, "hidden_activation": "gelu_pytorch_tanh", "max_position_embeddings": 256,
        "rms_norm_eps": cfg.eps, "tie_word_embeddings": True, "sliding_window": cfg.window,
        "layer_types": ["sliding_attention" if lay.sliding else "full_attention" for lay in cfg.layers],
        "final_logit_softcapping": cfg.softcap, "vocab_size_per_layer_input": cfg.ple_vocab,
        "hidden_size_per_layer_input": cfg.ple_dim, "num_kv_shared_layers": n_shared, "use_double_wide_mlp": True,
        "pad_token_id": 0, "bos_token_id": 2, "eos_token_id": 1,
        "rope_parameters": {"sliding_attention": {"rope_type": "default", "rope_theta": sl.rope_theta},
                            "full_attention": {"rope_type": "proportional",
                                               "partial_rotary_factor": 2 * fl.rope_pairs / fl.head_dim,
                                               "rope_theta": fl.rope_theta}},
    }


def hf_state(cfg: g4.G4Config, w: dict, prefix: str = "model.") -> dict[str, np.ndarray]:
    """transformers' tensor names -> the arrays of the converted-file weights w
    (wqkv split back into q/k/v, the layer scalars as [1] tensors)."""
    m = prefix
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
        sd[p + "layer_scalar"] = np.array([lay.layer_scalar], np.float32)
    return sd
