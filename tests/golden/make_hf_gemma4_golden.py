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
under transformers' names (tests/gemma4_hf.py): wqkv splits into q/k/v_proj
rows, the layer scalars become layer_scalar tensors.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import gemma4 as g4  # noqa: E402
from tests import gemma4_hf  # noqa: E402

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

    c = {k: v for k, v in gemma4_hf.text_config(cfg).items() if k != "model_type"}
    hc = Gemma4TextConfig(**c)
    hc._attn_implementation = "eager"
    model = Gemma4ForCausalLM(hc).to(torch.float64).eval()
    state = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in gemma4_hf.hf_state(cfg, w).items()}
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
