"""Write tests/golden/hf_gemma_tiny.npz: logits and greedy tokens of HF transformers'
GemmaForCausalLM (the reference's oracle dependency, ios_kernels/benchmarking/
reference.py:64-70) on a tiny Gemma-shaped config with the synthetic weights.

    python tests/golden/make_hf_gemma_golden.py

Runs in the build container only (it needs the locally installed transformers;
nothing is downloaded). The model is float64; weights are the hash-generator
values (fp16-representable), loaded by name: wqkv splits into q/k/v_proj rows
(fused order q|k|v, KL/convert_weights.py:9), RMSNorm weights are Gemma's
(1 + w) parameters, and the LM head is tied to the embedding.

The layer weights are N(0, 0.1^2) and the embedding N(0, 0.02^2): at the
common N(0, 0.02^2) the sqrt(D)-scaled embedding dominates this two-layer
model's residual stream and every greedy token repeats the last prompt id;
with these the 12 greedy tokens are all different (seed chosen for the widest
top-2 margin among seeds 11..30, 0.023).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import model as om  # noqa: E402

OUT = Path(__file__).resolve().parent / "hf_gemma_tiny.npz"
SEED = 29
STD = 0.1
EMBED_STD = 0.02
PROMPT = [5, 17, 999, 3, 250, 250, 42]
N_NEW = 12


def main() -> None:
    from transformers import GemmaConfig, GemmaForCausalLM

    cfg = om.TINY
    w = om.make_weights(cfg, SEED, STD, EMBED_STD)
    hc = GemmaConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.dim, intermediate_size=cfg.ffn_dim, num_hidden_layers=cfg.n_layers,
        num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads, head_dim=cfg.head_dim,
        hidden_activation="gelu_pytorch_tanh", rms_norm_eps=cfg.eps, rope_theta=cfg.rope_theta,
        max_position_embeddings=256, tie_word_embeddings=True, attention_bias=False, pad_token_id=0,
        bos_token_id=1, eos_token_id=2,
    )
    hc._attn_implementation = "eager"
    model = GemmaForCausalLM(hc).to(torch.float64).eval()
    hd, nh, nkv = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["final_norm"]}
    for l in range(cfg.n_layers):
        p = f"model.layers.{l}."
        qkv = w[f"l{l}.wqkv"]
        sd[p + "self_attn.q_proj.weight"] = qkv[: nh * hd]
        sd[p + "self_attn.k_proj.weight"] = qkv[nh * hd : (nh + nkv) * hd]
        sd[p + "self_attn.v_proj.weight"] = qkv[(nh + nkv) * hd :]
        sd[p + "self_attn.o_proj.weight"] = w[f"l{l}.wo"]
        sd[p + "mlp.gate_proj.weight"] = w[f"l{l}.wgate"]
        sd[p + "mlp.up_proj.weight"] = w[f"l{l}.wup"]
        sd[p + "mlp.down_proj.weight"] = w[f"l{l}.wdown"]
        sd[p + "input_layernorm.weight"] = w[f"l{l}.attn_norm"]
        sd[p + "post_attention_layernorm.weight"] = w[f"l{l}.ffn_norm"]
    state = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(state, strict=False)
    missing = [m for m in missing if m != "lm_head.weight"]
    assert not missing and not unexpected, (missing, unexpected)
    with torch.no_grad():
        logits = model(torch.tensor([PROMPT])).logits[0].numpy()
        gen = model.generate(torch.tensor([PROMPT]), max_new_tokens=N_NEW, do_sample=False, temperature=None,
                             top_p=None, top_k=None)[0, len(PROMPT):].tolist()
    np.savez_compressed(OUT, seed=SEED, std=STD, embed_std=EMBED_STD, prompt=np.array(PROMPT, np.int32),
                        logits=logits.astype(np.float64), greedy=np.array(gen, np.int32))
    print(f"wrote {OUT}: logits {logits.shape}, greedy {gen}")


if __name__ == "__main__":
    main()
