"""Gemma-4 host logic without a GPU: the per-layer facts resolved from an HF
text config (KG/convert_weights.py engine_config) against the oracle's, the
streamed-bytes count of the E2B shape (KG/PLAN.md: 4.56 GB per token), and
the engine's rejection of inconsistent layers before any device work."""

from __future__ import annotations

import pytest

from oracle import gemma4 as g4


def _layers_equal(a, b):
    return [(y.head_dim, y.ffn_dim, y.sliding, y.kv_layer, y.rope_pairs, y.rope_theta) for y in a] == \
           [(y.head_dim, y.ffn_dim, y.sliding, y.kv_layer, y.rope_pairs, y.rope_theta) for y in b]


def test_e2b_layers_match_oracle():
    from gemmagemini4hackathon2026_10_2425_amd.engine import GEMMA4_E2B

    assert _layers_equal(GEMMA4_E2B.layers, g4.G4_E2B.layers)
    assert (GEMMA4_E2B.dim, GEMMA4_E2B.n_heads, GEMMA4_E2B.n_kv_heads, GEMMA4_E2B.vocab, GEMMA4_E2B.ple_dim,
            GEMMA4_E2B.window) == (1536, 8, 1, 262144, 256, 512)
    # KV sharing: layers 15-34 read layer 13 (sliding) or 14 (full)
    assert {y.kv_layer for y in GEMMA4_E2B.layers[15:]} == {13, 14}
    # 2.28 B streamed parameters = 4.56 GB in fp16 per decoded token
    assert abs(GEMMA4_E2B.weight_bytes / 1e9 - 4.56) < 0.01


def test_tiny_layers_from_hf_config():
    from gemmagemini4hackathon2026_10_2425_amd.engine import Gemma4Shape

    c = {"hidden_size": 256, "num_hidden_layers": 6, "num_attention_heads": 4, "num_key_value_heads": 1,
         "head_dim": 64, "global_head_dim": 128, "intermediate_size": 512, "vocab_size": 1000,
         "hidden_size_per_layer_input": 32, "sliding_window": 16, "final_logit_softcapping": 30.0,
         "num_kv_shared_layers": 2, "use_double_wide_mlp": True, "layer_types": g4.G4_TINY_TYPES,
         "rope_parameters": {"sliding_attention": {"rope_type": "default", "rope_theta": 10000.0},
                             "full_attention": {"rope_type": "proportional", "partial_rotary_factor": 0.25,
                                                "rope_theta": 1000000.0}}}
    s = Gemma4Shape.from_hf(c)
    assert _layers_equal(s.layers, g4.G4_TINY.layers)
    assert s.softcap == 30.0 and s.ple_vocab == 1000
    bad = dict(c, rope_parameters={**c["rope_parameters"], "full_attention": {"rope_type": "yarn", "rope_theta": 1.0}})
    with pytest.raises(ValueError, match="rope type"):
        Gemma4Shape.from_hf(bad)
    with pytest.raises(ValueError, match="dense"):
        Gemma4Shape.from_hf(dict(c, enable_moe_block=True))


def _tiny_shape():
    from gemmagemini4hackathon2026_10_2425_amd.engine import Gemma4Layer, Gemma4Shape

    cfg = g4.G4_TINY
    layers = tuple(Gemma4Layer(y.head_dim, y.ffn_dim, y.sliding, y.kv_layer, y.rope_pairs, y.rope_theta,
                               y.layer_scalar) for y in cfg.layers)
    return Gemma4Shape(cfg.dim, cfg.n_heads, 1, cfg.vocab, cfg.ple_dim, cfg.ple_vocab, cfg.window, layers)


def test_engine_rejects_bad_layers():
    from gemmagemini4hackathon2026_10_2425_amd import _lib
    from gemmagemini4hackathon2026_10_2425_amd.engine import Engine, Gemma4Layer, Gemma4Shape

    base = _tiny_shape()
    L = base.layers
    bad = {
        "head_dim": L[:4] + (Gemma4Layer(96, 512, True, 4, 16, 1e4),) + L[5:],
        "same head_dim": L[:4] + (Gemma4Layer(64, 512, True, 2, 32, 1e4),) + L[5:],
        "earlier layer": L[:1] + (Gemma4Layer(64, 512, True, 3, 32, 1e4),) + L[2:],
        "rope_pairs": L[:1] + (Gemma4Layer(64, 512, True, 1, 33, 1e4),) + L[2:],
    }
    for what, layers in bad.items():
        shape = Gemma4Shape(base.dim, base.n_heads, 1, base.vocab, base.ple_dim, base.ple_vocab, base.window, layers)
        with pytest.raises(_lib.MxdValueError):
            Engine(shape, 64)
    with pytest.raises(_lib.MxdValueError, match="group size"):
        Engine(Gemma4Shape(base.dim, 3, 1, base.vocab, base.ple_dim, base.ple_vocab, base.window, L), 64)
    with pytest.raises(_lib.MxdValueError, match="max_ctx"):
        Engine(base, 48)


def _g4_snapshot(d, cfg, w, multimodal: bool):
    """A local HF checkpoint directory of the oracle's weights: a text-only
    Gemma4ForCausalLM layout, or the multimodal one (text model under
    model.language_model., config under text_config)."""
    import json

    import numpy as np
    import torch
    from safetensors.torch import save_file

    from tests import gemma4_hf

    text = gemma4_hf.text_config(cfg)
    sd = gemma4_hf.hf_state(cfg, w, "model.language_model." if multimodal else "model.")
    d.mkdir(parents=True, exist_ok=True)
    save_file({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}, str(d / "model.safetensors"))
    config = {"model_type": "gemma4", "text_config": text} if multimodal else text
    (d / "config.json").write_text(json.dumps(config))
    return text


@pytest.mark.parametrize("multimodal", [False, True])
def test_convert_gemma4_checkpoint(tmp_path, multimodal):
    """The converter writes the reference's Gemma-4 file (KG/convert_weights.py):
    the text config, the resolved per-layer facts with the checkpoint's layer
    scalars, and every tensor bit for bit; the loader reads the shape back."""
    import numpy as np

    from gemmagemini4hackathon2026_10_2425_amd import weights as W

    cfg = g4.G4_TINY
    w = g4.make_weights(cfg, 5)
    text = _g4_snapshot(tmp_path / "snap", cfg, w, multimodal)
    W.convert_hf(tmp_path / "snap", tmp_path / "g4.bin")
    header, t = W.read_bin_full(tmp_path / "g4.bin")
    assert header["config"] == text
    assert [y["layer_scalar"] for y in header["engine"]["layers"]] == \
           [float(np.float32(y.layer_scalar)) for y in cfg.layers]
    shape = W.gemma4_shape(header["config"], header["engine"])
    assert _layers_equal(shape.layers, cfg.layers)
    assert [y.layer_scalar for y in shape.layers] == [float(np.float32(y.layer_scalar)) for y in cfg.layers]
    assert list(t) == W.gemma4_tensor_names(shape)
    assert sorted(t) == sorted(w)
    for name, a in w.items():
        assert t[name].dtype == a.dtype and np.array_equal(t[name].view(np.uint8), a.view(np.uint8)), name


def test_gemma4_file_needs_engine_header(tmp_path):
    import numpy as np

    from gemmagemini4hackathon2026_10_2425_amd import weights as W
    from tests import gemma4_hf

    W.write_bin(tmp_path / "x.bin", gemma4_hf.text_config(g4.G4_TINY), {"embed": np.zeros((4, 4), np.float16)})
    with pytest.raises(ValueError, match="engine"):
        W.load_engine(tmp_path / "x.bin", 64)
