"""The reference's flat weight file, read into the engine and written from host
arrays or a local HF checkpoint.

Format (writer KL/convert_weights.py:1-11,71-89; reader KL/main.swift:113-140):

    [0:8)     little-endian u64 header length H
    [8:8+H)   UTF-8 JSON {"config": {HF config.json}, "tensors": {name: {"offset", "shape", "dtype"}}}
    ...       tensor data at absolute offsets, each on a 256-byte boundary
    the file is padded to a multiple of 16 KiB

Tensor names (KL/convert_weights.py:56-69): embed, l<i>.attn_norm, l<i>.wqkv
(rows q | k | v), l<i>.wo, l<i>.ffn_norm, l<i>.wgate, l<i>.wup, l<i>.wdown,
final_norm, and lm_head when the head is not tied. Norm weights are fp32,
everything else fp16.

A Gemma-4 file (KG/convert_weights.py:1-15) has the same layout; its header
adds "engine": {"layers": [{head_dim, ffn_dim, sliding, kv_layer, rope_theta,
rope_pairs, layer_scalar}]}, "config" is the checkpoint's text config, and the
tensors are embed, ple_embed, ple_proj, ple_norm, per layer attn_norm, wqkv
(q only on KV-shared layers), q_norm, k_norm (own K/V only), wo,
post_attn_norm, ffn_norm, wgate, wup, wdown, post_ffn_norm, ple_gate,
ple_out, post_ple_norm, and final_norm.

The engine covers Gemma-1/2B-style and Llama-style decoders (Llama-3.2-1B
included) with a tied or untied LM head, head_dim 64, 128 or 256, and plain or
Llama-3-scaled RoPE, and Gemma-4 (E2B-style) text models; a file outside that
raises ValueError naming what is unsupported.
"""

from __future__ import annotations

import glob
import json
import os
from pathlib import Path

import numpy as np

from .engine import Engine, Gemma4Layer, Gemma4Shape, ModelShape

ALIGN = 256
PAGE = 16384
HEADER_RESERVE = 64 * 1024  # the reference writer's fixed header prefix
_DTYPES = {"float16": np.float16, "float32": np.float32}
_LAYER_KINDS = ("attn_norm", "wqkv", "wo", "ffn_norm", "wgate", "wup", "wdown")


# ---------------------------------------------------------------- file format


def write_bin(path: str | os.PathLike, config: dict, tensors: dict[str, np.ndarray], engine: dict | None = None) -> int:
    """Write `tensors` (name -> fp16/fp32 array, in the given order) and the
    model config (and a Gemma-4 file's "engine" facts) in the flat format.
    Returns the file size in bytes."""
    arrays = []
    for name, arr in tensors.items():
        a = np.ascontiguousarray(arr)
        if a.dtype not in (np.float16, np.float32):
            raise ValueError(f"{name}: dtype {a.dtype} (float16 or float32)")
        arrays.append((name, a))
    start = HEADER_RESERVE
    while True:  # the header's own length decides where the data can start
        off, meta = start, {}
        for name, a in arrays:
            off = (off + ALIGN - 1) // ALIGN * ALIGN
            meta[name] = {"offset": off, "shape": list(a.shape), "dtype": str(a.dtype)}
            off += a.nbytes
        head = {"config": config, "tensors": meta}
        if engine is not None:
            head = {"config": config, "engine": engine, "tensors": meta}
        header = json.dumps(head).encode()
        if 8 + len(header) <= start:
            break
        start = (8 + len(header) + ALIGN - 1) // ALIGN * ALIGN
    total = (off + PAGE - 1) // PAGE * PAGE
    with open(path, "wb") as f:
        f.write(len(header).to_bytes(8, "little"))
        f.write(header)
        for name, a in arrays:
            f.seek(meta[name]["offset"])
            f.write(a.tobytes())
        f.truncate(total)
    return total


def read_bin(path: str | os.PathLike) -> tuple[dict, dict[str, np.ndarray]]:
    """(config, {name: read-only array over a memory map of the file})."""
    header, tensors = read_bin_full(path)
    return header["config"], tensors


def read_bin_full(path: str | os.PathLike) -> tuple[dict, dict[str, np.ndarray]]:
    """(the whole JSON header, {name: read-only array over a memory map})."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) < 8:
            raise ValueError(f"{path}: not a weight file (shorter than its 8-byte header length)")
        hlen = int.from_bytes(head, "little")
        if hlen <= 0 or 8 + hlen > size:
            raise ValueError(f"{path}: header length {hlen} does not fit a file of {size} bytes")
        header = json.loads(f.read(hlen).decode())
    if "config" not in header or "tensors" not in header:
        raise ValueError(f"{path}: header lacks 'config' or 'tensors'")
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    tensors = {}
    for name, m in header["tensors"].items():
        dt = _DTYPES.get(m.get("dtype"))
        if dt is None:
            raise ValueError(f"{path}: tensor {name} has dtype {m.get('dtype')!r} (float16 or float32)")
        shape = tuple(int(s) for s in m["shape"])
        off, nb = int(m["offset"]), int(np.prod(shape, dtype=np.int64)) * np.dtype(dt).itemsize
        if off < 8 + hlen or off + nb > size:
            raise ValueError(f"{path}: tensor {name} [{off}, {off + nb}) lies outside the data region")
        tensors[name] = mm[off : off + nb].view(dt).reshape(shape)
    return header, tensors


# ---------------------------------------------------------------- config


def _rope(c: dict) -> tuple[float, tuple | None]:
    """(rope_theta, Llama-3 scaling or None) of a config: transformers 4.x
    writes rope_theta and rope_scaling at the top level, 5.x both inside
    rope_parameters. rope_type "default" is plain RoPE, "llama3" the band
    scaling of KL/main.swift:96-107; any other type is rejected."""
    rp = c.get("rope_parameters") or {}
    theta = c.get("rope_theta", rp.get("rope_theta", 10000.0))
    scaling = c.get("rope_scaling") or (rp if rp.get("rope_type", "default") != "default" else None)
    if not scaling:
        return float(theta), None
    rtype = scaling.get("rope_type", scaling.get("type"))
    if rtype == "default":
        return float(theta), None
    if rtype != "llama3":
        raise ValueError(f"rope scaling {scaling!r} is not supported (default or llama3)")
    try:
        return float(theta), (float(scaling["factor"]), float(scaling["low_freq_factor"]),
                               float(scaling["high_freq_factor"]), int(scaling["original_max_position_embeddings"]))
    except KeyError as err:
        raise ValueError(f"llama3 rope scaling lacks {err}") from None


def shape_from_config(c: dict) -> ModelShape:
    """ModelShape of an HF-style config (the keys KL/main.swift:75-110 reads).
    model_type "gemma": GeGLU (tanh), (1 + w) RMSNorm, sqrt(D) embedding scale.
    "llama" (and configs without a model_type): SwiGLU, w RMSNorm, no scale.
    tie_word_embeddings false means a separate lm_head tensor (KL/main.swift:306)."""
    mt = c.get("model_type", "llama")
    if mt not in ("gemma", "llama"):
        raise ValueError(f"model_type {mt!r} is not supported (gemma or llama)")
    theta, scaling = _rope(c)
    if c.get("attention_bias") or c.get("mlp_bias"):
        raise ValueError("projection biases are not supported")
    tied = bool(c.get("tie_word_embeddings", mt == "gemma"))
    act = c.get("hidden_activation") or c.get("hidden_act") or ("gelu_pytorch_tanh" if mt == "gemma" else "silu")
    if act in ("gelu_pytorch_tanh", "gelu_tanh") or (mt == "gemma" and act == "gelu"):
        act = "gelu_tanh"  # Gemma's "gelu" is the tanh form (KG/kernels.metal:26-28)
    elif act != "silu":
        raise ValueError(f"activation {act!r} is not supported (gelu_pytorch_tanh or silu)")
    dim, nh = int(c["hidden_size"]), int(c["num_attention_heads"])
    gemma = mt == "gemma"
    return ModelShape(
        n_layers=int(c["num_hidden_layers"]), dim=dim, n_heads=nh,
        n_kv_heads=int(c.get("num_key_value_heads", nh)), head_dim=int(c.get("head_dim") or dim // nh),
        ffn_dim=int(c["intermediate_size"]), vocab=int(c["vocab_size"]),
        rms_eps=float(c.get("rms_norm_eps", 1e-6)), rope_theta=theta, act=act,
        norm_plus_one=gemma, embed_scale_sqrt_dim=gemma, tie_embeddings=tied, rope_scaling=scaling,
    )


def tensor_names(n_layers: int, tied: bool = True) -> list[str]:
    names = ["embed"] + [f"l{i}.{k}" for i in range(n_layers) for k in _LAYER_KINDS] + ["final_norm"]
    return names if tied else names + ["lm_head"]


def is_gemma4(config: dict) -> bool:
    """A Gemma-4 config: model_type gemma4 / gemma4_text, or a text_config of one."""
    mt = str(config.get("model_type", ""))
    return mt.startswith("gemma4") or str((config.get("text_config") or {}).get("model_type", "")).startswith("gemma4")


def gemma4_shape(config: dict, engine: dict | None = None) -> Gemma4Shape:
    """Gemma4Shape of a text config; the per-layer facts from a file's "engine"
    header when given (KG/main.swift:86-101), else resolved from the config
    (layer scalars 1)."""
    text = config.get("text_config", config)
    layers = None
    if engine is not None:
        try:
            layers = tuple(Gemma4Layer(int(y["head_dim"]), int(y["ffn_dim"]), bool(y["sliding"]), int(y["kv_layer"]),
                                       int(y["rope_pairs"]), float(y["rope_theta"]),
                                       float(y.get("layer_scalar", 1.0))) for y in engine["layers"])
        except (KeyError, TypeError) as err:
            raise ValueError(f"engine header: bad layer entry ({err})") from None
        if len(layers) != int(text["num_hidden_layers"]):
            raise ValueError(f"engine header has {len(layers)} layers for num_hidden_layers "
                             f"{text['num_hidden_layers']}")
    return Gemma4Shape.from_hf(text, layers)


def gemma4_tensor_names(shape: Gemma4Shape) -> list[str]:
    """Tensor names of a Gemma-4 file, in the reference converter's order
    (KG/convert_weights.py:98-121)."""
    names = ["embed", "ple_embed", "ple_proj", "ple_norm"]
    for i, y in enumerate(shape.layers):
        own = y.kv_layer == i
        names += [f"l{i}.{k}" for k in ("attn_norm", "wqkv", "q_norm") + (("k_norm",) if own else ()) +
                  ("wo", "post_attn_norm", "ffn_norm", "wgate", "wup", "wdown", "post_ffn_norm", "ple_gate",
                   "ple_out", "post_ple_norm")]
    return names + ["final_norm"]


# ---------------------------------------------------------------- engine


def load_engine(path: str | os.PathLike, max_ctx: int = 4096) -> Engine:
    """An Engine holding the file's weights (every tensor checked for name,
    dtype and size before the first upload)."""
    header, tensors = read_bin_full(path)
    config = header["config"]
    if "engine" in header or is_gemma4(config):
        if "engine" not in header:
            raise ValueError(f"{path}: a Gemma-4 file needs the 'engine' header (KG/convert_weights.py)")
        shape = gemma4_shape(config, header["engine"])
        names = gemma4_tensor_names(shape)
    else:
        shape = shape_from_config(config)
        names = tensor_names(shape.n_layers, shape.tie_embeddings)
    extra = sorted(set(tensors) - set(names))
    if extra:
        raise ValueError(f"{path}: tensors the engine does not use: {', '.join(extra[:8])}")
    e = Engine(shape, max_ctx)
    try:
        want = {name: (nb, dt) for name, nb, dt in e.tensor_specs()}
        for name, (nb, dt) in want.items():
            if name not in tensors:
                raise ValueError(f"{path}: missing tensor {name}")
            a = tensors[name]
            if a.dtype != dt or a.nbytes != nb:
                raise ValueError(f"{path}: {name} is {a.dtype} {list(a.shape)} ({a.nbytes} B); "
                                 f"the engine needs {np.dtype(dt).name} of {nb} B")
        for name in want:
            e.upload(name, tensors[name])
    except BaseException:
        e.close()
        raise
    return e


# ---------------------------------------------------------------- conversion


def _snapshot(repo: str) -> Path:
    """The local HF cache snapshot of `repo` (no download), as
    KL/convert_weights.py:25-30 finds it."""
    base = Path(os.path.expanduser("~/.cache/huggingface/hub")) / f"models--{repo.replace('/', '--')}" / "snapshots"
    for snap in sorted(glob.glob(str(base / "*"))):
        if glob.glob(os.path.join(snap, "*.safetensors")):
            return Path(snap)
    raise FileNotFoundError(f"no *.safetensors under {base}")


def convert_hf(src: str | os.PathLike, out: str | os.PathLike) -> int:
    """Convert a local HF checkpoint directory (config.json + *.safetensors) to
    the flat file, as KL/convert_weights.py:33-69 does: q|k|v fused per layer,
    norms fp32, the rest fp16 (checked for fp16 overflow). Returns the size."""
    from safetensors import safe_open

    src = Path(src)
    config = json.loads((src / "config.json").read_text())
    gemma4 = is_gemma4(config)
    # reject what the engine cannot run before converting
    shape = gemma4_shape(config) if gemma4 else shape_from_config(config)
    files = sorted(src.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {src}")
    where = {}
    for fpath in files:
        with safe_open(str(fpath), "pt") as st:
            for k in st.keys():
                where[k] = fpath

    def get(name: str) -> np.ndarray:
        if name not in where:
            raise KeyError(f"{src}: checkpoint has no tensor {name}")
        with safe_open(str(where[name]), "pt") as st:
            return st.get_tensor(name).float().numpy()

    def f16(name: str, a: np.ndarray) -> np.ndarray:
        m = float(np.abs(a).max()) if a.size else 0.0
        if m >= 65504:
            raise ValueError(f"{name} overflows fp16 (max |w| = {m})")
        return a.astype(np.float16)

    if gemma4:
        return _convert_gemma4(config, shape, where, get, f16, out)
    out_t: dict[str, np.ndarray] = {"embed": f16("embed", get("model.embed_tokens.weight"))}
    for i in range(int(config["num_hidden_layers"])):
        p = f"model.layers.{i}."
        out_t[f"l{i}.attn_norm"] = get(p + "input_layernorm.weight").astype(np.float32)
        qkv = np.concatenate([get(p + f"self_attn.{n}_proj.weight") for n in "qkv"], axis=0)
        out_t[f"l{i}.wqkv"] = f16(f"l{i}.wqkv", qkv)
        out_t[f"l{i}.wo"] = f16(f"l{i}.wo", get(p + "self_attn.o_proj.weight"))
        out_t[f"l{i}.ffn_norm"] = get(p + "post_attention_layernorm.weight").astype(np.float32)
        out_t[f"l{i}.wgate"] = f16(f"l{i}.wgate", get(p + "mlp.gate_proj.weight"))
        out_t[f"l{i}.wup"] = f16(f"l{i}.wup", get(p + "mlp.up_proj.weight"))
        out_t[f"l{i}.wdown"] = f16(f"l{i}.wdown", get(p + "mlp.down_proj.weight"))
    out_t["final_norm"] = get("model.norm.weight").astype(np.float32)
    if not shape.tie_embeddings:
        out_t["lm_head"] = f16("lm_head", get("lm_head.weight"))
    return write_bin(out, config, out_t)


def _convert_gemma4(config: dict, shape: Gemma4Shape, where: dict, get, f16, out) -> int:
    """The text model of a Gemma-4 checkpoint as KG/convert_weights.py:73-144
    writes it: the per-layer facts in the "engine" header (layer_scalar read
    from the checkpoint), q|k|v fused (q only on KV-shared layers), norms fp32,
    the rest fp16. Tensors live under model.language_model. (the multimodal
    checkpoint) or model. (a text-only one)."""
    text = config.get("text_config", config)
    if not text.get("tie_word_embeddings", True):
        raise ValueError("the Gemma-4 LM head is the tied embedding (tie_word_embeddings false is not supported)")
    pre = "model.language_model." if "model.language_model.embed_tokens.weight" in where else "model."
    f32 = lambda name: get(pre + name).astype(np.float32)  # noqa: E731
    out_t: dict[str, np.ndarray] = {
        "embed": f16("embed", get(pre + "embed_tokens.weight")),
        "ple_embed": f16("ple_embed", get(pre + "embed_tokens_per_layer.weight")),
        "ple_proj": f16("ple_proj", get(pre + "per_layer_model_projection.weight")),
        "ple_norm": f32("per_layer_projection_norm.weight"),
    }
    layers = []
    for i, y in enumerate(shape.layers):
        p = f"layers.{i}."
        own = y.kv_layer == i
        scalar = float(get(pre + p + "layer_scalar").reshape(-1)[0])
        layers.append({"head_dim": y.head_dim, "ffn_dim": y.ffn_dim, "sliding": y.sliding, "kv_layer": y.kv_layer,
                       "rope_theta": y.rope_theta, "rope_pairs": y.rope_pairs, "layer_scalar": scalar})
        out_t[f"l{i}.attn_norm"] = f32(p + "input_layernorm.weight")
        qkv = [get(pre + p + f"self_attn.{n}_proj.weight") for n in ("qkv" if own else "q")]
        out_t[f"l{i}.wqkv"] = f16(f"l{i}.wqkv", np.concatenate(qkv, axis=0))
        out_t[f"l{i}.q_norm"] = f32(p + "self_attn.q_norm.weight")
        if own:
            out_t[f"l{i}.k_norm"] = f32(p + "self_attn.k_norm.weight")
        out_t[f"l{i}.wo"] = f16(f"l{i}.wo", get(pre + p + "self_attn.o_proj.weight"))
        out_t[f"l{i}.post_attn_norm"] = f32(p + "post_attention_layernorm.weight")
        out_t[f"l{i}.ffn_norm"] = f32(p + "pre_feedforward_layernorm.weight")
        out_t[f"l{i}.wgate"] = f16(f"l{i}.wgate", get(pre + p + "mlp.gate_proj.weight"))
        out_t[f"l{i}.wup"] = f16(f"l{i}.wup", get(pre + p + "mlp.up_proj.weight"))
        out_t[f"l{i}.wdown"] = f16(f"l{i}.wdown", get(pre + p + "mlp.down_proj.weight"))
        out_t[f"l{i}.post_ffn_norm"] = f32(p + "post_feedforward_layernorm.weight")
        out_t[f"l{i}.ple_gate"] = f16(f"l{i}.ple_gate", get(pre + p + "per_layer_input_gate.weight"))
        out_t[f"l{i}.ple_out"] = f16(f"l{i}.ple_out", get(pre + p + "per_layer_projection.weight"))
        out_t[f"l{i}.post_ple_norm"] = f32(p + "post_per_layer_input_norm.weight")
    out_t["final_norm"] = f32("norm.weight")
    return write_bin(out, text, out_t, engine={"layers": layers})


def main(argv=None) -> int:
    """convert script of the kernel folder contract: --repo <hf_repo> | --src DIR, --out PATH."""
    import argparse

    ap = argparse.ArgumentParser(description="HF checkpoint -> flat fp16 weight file")
    g = ap.add_mutually_exclusive_group(required=True)
    g.add_argument("--repo", help="HF repo id, read from the local HF cache (nothing is downloaded)")
    g.add_argument("--src", help="a local directory with config.json and *.safetensors")
    ap.add_argument("--out", required=True)
    args = ap.parse_args(argv)
    src = Path(args.src) if args.src else _snapshot(args.repo)
    total = convert_hf(src, args.out)
    print(f"wrote {args.out}: {total / 1e9:.3f} GB")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
