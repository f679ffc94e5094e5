"""Host side of the drop-in surface, on the CPU: the reference's flat weight
file (writer KL/convert_weights.py:71-89, reader KL/main.swift:113-140), the HF
config mapping, the HF-checkpoint converter, the engine binary's options and
the --serve protocol (KL/main.swift:494-547) over a stand-in engine."""

from __future__ import annotations

import io
import json
import os
import stat
from pathlib import Path

import numpy as np
import pytest

from oracle import model as om

PKG = Path(__file__).resolve().parents[1] / "gemmagemini4hackathon2026_10_2425_amd"


def _w():
    from gemmagemini4hackathon2026_10_2425_amd import weights

    return weights


GEMMA_TINY_CFG = {
    "model_type": "gemma", "vocab_size": om.TINY.vocab, "hidden_size": om.TINY.dim,
    "intermediate_size": om.TINY.ffn_dim, "num_hidden_layers": om.TINY.n_layers,
    "num_attention_heads": om.TINY.n_heads, "num_key_value_heads": om.TINY.n_kv_heads,
    "head_dim": om.TINY.head_dim, "hidden_activation": "gelu_pytorch_tanh", "rms_norm_eps": om.TINY.eps,
    "rope_theta": om.TINY.rope_theta, "tie_word_embeddings": True,
}


def test_bin_round_trip_and_layout(tmp_path):
    W = _w()
    w = om.make_weights(om.TINY, 3)
    path = tmp_path / "m.bin"
    total = W.write_bin(path, GEMMA_TINY_CFG, w)
    raw = path.read_bytes()
    assert len(raw) == total and total % W.PAGE == 0
    hlen = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8 : 8 + hlen])
    assert header["config"] == GEMMA_TINY_CFG
    assert list(header["tensors"]) == list(w)  # file order = writer order
    for name, m in header["tensors"].items():
        assert m["offset"] % W.ALIGN == 0 and m["offset"] >= W.HEADER_RESERVE
        assert m["dtype"] == str(w[name].dtype) and m["shape"] == list(w[name].shape)
        # absolute offsets: the bytes at the offset are the tensor's bytes
        assert raw[m["offset"] : m["offset"] + w[name].nbytes] == w[name].tobytes(), name
    cfg, t = W.read_bin(path)
    assert cfg == GEMMA_TINY_CFG
    for name, a in w.items():
        assert t[name].dtype == a.dtype and np.array_equal(t[name].view(np.uint8), a.view(np.uint8)), name


def test_bin_large_header(tmp_path):
    """A header longer than the 64 KiB prefix moves the data start."""
    W = _w()
    cfg = dict(GEMMA_TINY_CFG, notes="x" * 70000)
    w = {"embed": np.ones((4, 8), np.float16), "final_norm": np.arange(8, dtype=np.float32)}
    W.write_bin(tmp_path / "h.bin", cfg, w)
    c2, t = W.read_bin(tmp_path / "h.bin")
    assert c2["notes"] == cfg["notes"] and np.array_equal(t["final_norm"], w["final_norm"])


def test_read_bin_rejects_bad_files(tmp_path):
    W = _w()
    (tmp_path / "short.bin").write_bytes(b"\x01\x02")
    with pytest.raises(ValueError):
        W.read_bin(tmp_path / "short.bin")
    (tmp_path / "len.bin").write_bytes((1 << 40).to_bytes(8, "little") + b"{}")
    with pytest.raises(ValueError):
        W.read_bin(tmp_path / "len.bin")
    hdr = json.dumps({"config": {}, "tensors": {"embed": {"offset": 4096, "shape": [1000], "dtype": "float16"}}}).encode()
    (tmp_path / "oob.bin").write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 100)
    with pytest.raises(ValueError, match="outside"):
        W.read_bin(tmp_path / "oob.bin")
    hdr = json.dumps({"config": {}, "tensors": {"e": {"offset": 256, "shape": [2], "dtype": "bfloat16"}}}).encode()
    (tmp_path / "dt.bin").write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 600)
    with pytest.raises(ValueError, match="dtype"):
        W.read_bin(tmp_path / "dt.bin")


def test_shape_from_config():
    W = _w()
    s = W.shape_from_config(GEMMA_TINY_CFG)
    assert (s.n_layers, s.dim, s.n_heads, s.n_kv_heads, s.head_dim, s.ffn_dim, s.vocab) == (
        om.TINY.n_layers, om.TINY.dim, om.TINY.n_heads, om.TINY.n_kv_heads, om.TINY.head_dim, om.TINY.ffn_dim,
        om.TINY.vocab)
    assert s.act == "gelu_tanh" and s.norm_plus_one and s.embed_scale_sqrt_dim
    # Gemma-1 configs say hidden_act "gelu" and mean the tanh form
    assert W.shape_from_config(dict(GEMMA_TINY_CFG, hidden_activation=None, hidden_act="gelu")).act == "gelu_tanh"
    llama = {"model_type": "llama", "vocab_size": 3000, "hidden_size": 512, "intermediate_size": 1024,
             "num_hidden_layers": 3, "num_attention_heads": 4, "num_key_value_heads": 2, "hidden_act": "silu",
             "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "tie_word_embeddings": True}
    s = W.shape_from_config(llama)
    assert s.head_dim == 128 and s.act == "silu" and not s.norm_plus_one and not s.embed_scale_sqrt_dim
    assert s.rms_eps == 1e-5 and s.rope_theta == 500000.0
    assert s.tie_embeddings and s.rope_scaling is None
    assert not W.shape_from_config(dict(llama, tie_word_embeddings=False)).tie_embeddings
    l3 = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    assert W.shape_from_config(dict(llama, rope_scaling=l3)).rope_scaling == (32.0, 1.0, 4.0, 8192)
    for bad, msg in [({"rope_scaling": {"rope_type": "llama3", "factor": 32.0}}, "lacks"),
                     ({"rope_scaling": {"rope_type": "yarn", "factor": 4.0}}, "not supported"),
                     ({"model_type": "gemma3"}, "model_type"),
                     ({"hidden_act": "relu"}, "activation"), ({"attention_bias": True}, "bias")]:
        with pytest.raises(ValueError, match=msg):
            W.shape_from_config(dict(llama, **bad))


def test_shape_from_transformers5_configs():
    """transformers 5.x keeps rope_theta and the scaling inside rope_parameters
    (the layout of every checkpoint the installed version saves); a Llama-3.2-1B
    config maps to the engine's Llama-3.2-1B shape."""
    from transformers import LlamaConfig

    from gemmagemini4hackathon2026_10_2425_amd.engine import LLAMA32_1B

    W = _w()
    rp = {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 32.0, "low_freq_factor": 1.0,
          "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    hc = LlamaConfig(vocab_size=128256, hidden_size=2048, intermediate_size=8192, num_hidden_layers=16,
                     num_attention_heads=32, num_key_value_heads=8, head_dim=64, rms_norm_eps=1e-5,
                     max_position_embeddings=131072, tie_word_embeddings=True, rope_parameters=rp).to_dict()
    assert "rope_theta" not in hc  # the layout this test is about
    assert W.shape_from_config(hc) == LLAMA32_1B
    plain = LlamaConfig(hidden_size=512, intermediate_size=1024, num_attention_heads=4, num_hidden_layers=1,
                        rope_parameters={"rope_type": "default", "rope_theta": 250000.0}).to_dict()
    s = W.shape_from_config(plain)
    assert s.rope_theta == 250000.0 and s.rope_scaling is None
    yarn = dict(plain, rope_parameters={"rope_type": "yarn", "rope_theta": 1e4, "factor": 4.0})
    with pytest.raises(ValueError, match="not supported"):
        W.shape_from_config(yarn)


def _hf_snapshot(d: Path, cfg, seed: int, bf16_norms: bool = False, std: float = 0.02,
                 embed_std: float | None = None) -> dict:
    """A local HF-layout checkpoint (config.json + model.safetensors) whose
    tensors are the oracle's synthetic weights split back into q/k/v."""
    import torch
    from safetensors.torch import save_file

    w = om.make_weights(cfg, seed, std, embed_std)
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
    tens = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}
    if bf16_norms:  # bf16 storage as real checkpoints have it (values here are bf16-exact: 0)
        tens["model.layers.0.input_layernorm.weight"] = torch.zeros(cfg.dim, dtype=torch.bfloat16)
        w["l0.attn_norm"] = np.zeros(cfg.dim, np.float32)
    d.mkdir(parents=True, exist_ok=True)
    save_file(tens, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps(GEMMA_TINY_CFG))
    return w


def test_convert_hf_checkpoint(tmp_path):
    W = _w()
    w = _hf_snapshot(tmp_path / "snap", om.TINY, 11, bf16_norms=True)
    W.convert_hf(tmp_path / "snap", tmp_path / "g.bin")
    cfg, t = W.read_bin(tmp_path / "g.bin")
    assert cfg == GEMMA_TINY_CFG
    assert sorted(t) == sorted(W.tensor_names(om.TINY.n_layers))
    for name, a in w.items():
        assert t[name].dtype == a.dtype and np.array_equal(t[name].view(np.uint8), a.view(np.uint8)), name


def test_convert_rejects_fp16_overflow(tmp_path):
    import torch
    from safetensors.torch import save_file

    W = _w()
    _hf_snapshot(tmp_path / "snap", om.TINY, 1)
    from safetensors import safe_open

    with safe_open(str(tmp_path / "snap" / "model.safetensors"), "pt") as st:
        sd = {k: st.get_tensor(k) for k in st.keys()}
    sd["model.layers.1.mlp.up_proj.weight"] = sd["model.layers.1.mlp.up_proj.weight"].float() * 1e7
    save_file(sd, str(tmp_path / "snap" / "model.safetensors"))
    with pytest.raises(ValueError, match="overflows fp16"):
        W.convert_hf(tmp_path / "snap", tmp_path / "o.bin")


def test_kernel_folder_contract():
    """kernel.json names executable build / binary / convert files
    (ios_kernels/surfaces/DESIGN_AND_LIMITATIONS.md:70-79)."""
    d = PKG / "kernel"
    m = json.loads((d / "kernel.json").read_text())
    assert {"hf_repo", "weights", "build", "binary", "convert"} <= set(m)
    for key in ("build", "binary", "convert"):
        p = d / m[key]
        assert p.is_file() and os.stat(p).st_mode & stat.S_IXUSR, key
        assert p.read_text().startswith("#!/usr/bin/env python3")


# ---------------------------------------------------------------- engine binary


def test_cli_options():
    from gemmagemini4hackathon2026_10_2425_amd import serve

    a = serve.parse_args(["--weights", "w.bin", "--serve", "--max-ctx", "128", "--define", "MV_NR=8",
                          "--define", "ATT_WGCU=2", "--prompt-ids", "1,2,3", "--gen", "4", "--no-gemm"])
    assert a.serve and a.max_ctx == 128 and a.tunables == {"MV_NR": 8, "ATT_WGCU": 2} and a.ids == [1, 2, 3]
    assert a.gen == 4 and a.reps == 5
    for bad in (["--define", "MV_NR"], ["--define", "MV_NR=x"], ["--prompt-ids", "1,a"], ["--max-ctx", "100"],
                ["--bogus"], []):
        with pytest.raises(SystemExit):
            serve.parse_args((["--weights", "w.bin"] if bad != [] else []) + bad)


class _Shape:
    vocab = 50


class FakeEngine:
    """Stand-in with the engine's token semantics: prefill(n) writes
    tokens[n], each decode step at pos writes tokens[pos + 1]; the next token
    is (31 * previous + 7) mod vocab."""

    shape = _Shape()

    def __init__(self, max_ctx):
        self.t = [0] * (max_ctx + 1)
        self.steps = 0

    def _next(self, pos):
        self.t[pos + 1] = (31 * self.t[pos] + 7) % self.shape.vocab
        self.steps += 1

    def set_tokens(self, ids, start=0):
        self.t[start : start + len(ids)] = ids

    def prefill(self, n):
        self._next(n - 1)

    def decode(self, pos, count):
        for i in range(count):
            self._next(pos + i)

    def token(self, i):
        return self.t[i]

    def decode_streaming(self, pos, count, emit):
        for i in range(count):
            self._next(pos + i)
            if not emit(self.t[pos + i + 1]):
                return


def _chain(t0, n, vocab=50):
    out, t = [], t0
    for _ in range(n):
        t = (31 * t + 7) % vocab
        out.append(t)
    return out


def test_serve_protocol():
    from gemmagemini4hackathon2026_10_2425_amd import serve

    out = io.StringIO()
    srv = serve.Server(FakeEngine(64), 64, out, "test")
    srv.warmup()
    reqs = [
        json.dumps({"ids": [3, 4], "max_tokens": 5}),
        json.dumps({"ids": [3, 4], "max_tokens": 5, "stop_ids": [_chain(4, 5)[2]]}),
        "not json",
        json.dumps({"ids": []}),
        json.dumps({"ids": [1, 50]}),
        json.dumps({"ids": [1] * 64}),
        json.dumps({"ids": [1] * 60, "max_tokens": 100}),
        json.dumps({"ids": [9], "max_tokens": 0}),
        json.dumps({"ids": [True]}),
    ]
    srv.run(r + "\n" for r in reqs)
    lines = [json.loads(l) for l in out.getvalue().splitlines()]
    assert lines[0] == {"ready": True, "max_ctx": 64, "vocab": 50, "device": "test"}
    msgs = lines[1:]

    def take():
        toks = []
        while "token" in msgs[0]:
            toks.append(msgs.pop(0)["token"])
        return toks, msgs.pop(0)

    toks, done = take()
    assert toks == _chain(4, 5)
    assert done["done"] and done["finish_reason"] == "length" and done["prompt_tokens"] == 2
    assert done["completion_tokens"] == 5 and done["prefill_s"] >= 0 and done["decode_s"] >= 0
    toks, done = take()  # the stop token is not sent
    assert toks == _chain(4, 2) and done["finish_reason"] == "stop" and done["completion_tokens"] == 2
    for _ in range(2):  # not JSON, empty ids
        assert "expected" in msgs.pop(0)["error"]
    assert msgs.pop(0)["error"] == "token id 50 out of range"
    assert msgs.pop(0)["error"] == "prompt has 64 tokens, max_ctx is 64"
    toks, done = take()  # max_tokens clamped to max_ctx - prompt
    assert len(toks) == 4 and done["completion_tokens"] == 4 and done["finish_reason"] == "length"
    toks, done = take()
    assert toks == [] and done["completion_tokens"] == 0
    assert "expected" in msgs.pop(0)["error"]
    assert msgs == []


def test_generate_and_bench_formats(tmp_path):
    from gemmagemini4hackathon2026_10_2425_amd import serve

    e = FakeEngine(64)
    e.logits = lambda: np.arange(50, dtype=np.float32)
    e.tokens = lambda start, n: e.t[start : start + n]
    r = serve.generate(e, [5, 6, 7], 4, 64, str(tmp_path / "l.bin"))
    assert r["tokens"] == _chain(7, 4) and set(r) == {"tokens", "prefill_s", "decode_s", "decode_tok_s"}
    assert np.array_equal(np.fromfile(tmp_path / "l.bin", "<f4"), np.arange(50, dtype=np.float32))
    with pytest.raises(ValueError):
        serve.generate(e, [1] * 60, 5, 64)
    err = io.StringIO()
    rep = serve.bench(e, 8, 16, 2, {"MV_NR": 8}, err)
    assert rep["tunables"] == {"MV_NR": 8} and rep["pp"]["n"] == 8 and rep["tg"]["n"] == 16
    lines = err.getvalue().splitlines()
    import re

    assert re.match(r"^pp8: [\d.]+ ± [\d.]+ tok/s$", lines[0]) and re.match(r"^tg16: [\d.]+ ± [\d.]+ tok/s$", lines[1])
