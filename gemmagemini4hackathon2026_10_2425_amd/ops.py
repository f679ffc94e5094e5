"""Operator surface of the decode hot path on torch device tensors.

Names and argument meaning follow the reference's Metal operators (paths
relative to ios_kernels/kernels/, KL = the Llama-3.2-1B kernel folder,
KG = the Gemma-4-E2B kernel folder):

    matvec_f16 / matvec_f16_add / matvec_f16_gelu_mul   KG/kernels.metal:159-198
    matvec_q8b32                                        (new: int8 block-32)
    matvec_gate_up_gelu / matvec_gate_up_silu           KG/kernels.metal:205-234, KL/kernels.metal:144-173
    rmsnorm (rmsnorm_f32 / rmsnorm_f16)                 KL/kernels.metal:71-96
    embed / embed_rows                                  KL/kernels.metal:31-39, KG/kernels.metal:34-42
    rope_kv                                             KL/kernels.metal:182-224
    attention                                           KL/kernels.metal:235-305
    argmax                                              KL/kernels.metal:310-345
    f32_to_f16                                          KL/kernels.metal:361-365
    attention(window=) / attention_prefill(window=)     KG/kernels.metal:306-393
    rmsnorm_add                                         KG/kernels.metal:100-125
    ple_combine                                         KG/kernels.metal:127-149
    qk_norm_rope_kv (qkv_norm_rope)                     KG/kernels.metal:236-304

Every function checks shapes on the host and raises ValueError before any
launch (the reference's host preconditions, KG/main.swift:306, crash instead).
All work is enqueued on torch's current stream; tensors must live on the GPU.
torch is only the allocator/stream plumbing here: the arithmetic is in
libmxdecode.so.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib
from ._lib import call, query

_EPI = {"store": _lib.MXD_EPI_STORE, "add": _lib.MXD_EPI_ADD, "gelu_mul": _lib.MXD_EPI_GELU_MUL}
_ACT = {"gelu_tanh": _lib.MXD_ACT_GELU_TANH, "silu": _lib.MXD_ACT_SILU}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _on_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        _need(t.is_cuda, "tensor must be on the GPU")
        _need(t.is_contiguous(), "tensor must be contiguous")


def _xdtype(x: torch.Tensor) -> int:
    if x.dtype == torch.float32:
        return _lib.MXD_F32
    if x.dtype == torch.float16:
        return _lib.MXD_F16
    raise ValueError(f"activation dtype {x.dtype} (float32 or float16)")


# ---------------------------------------------------------------- weights


def fill_normal(shape, dtype: torch.dtype, seed: int, tensor_id: int, std: float, device="cuda") -> torch.Tensor:
    """Synthetic N(0, std^2) tensor from the counter-based generator (bit-exact
    with the oracle's restatement)."""
    _need(dtype in (torch.float32, torch.float16), "fill_normal: float32 or float16")
    t = torch.empty(shape, dtype=dtype, device=device)
    code = _lib.MXD_F32 if dtype == torch.float32 else _lib.MXD_F16
    call("mxd_fill_normal", _ptr(t), code, t.numel(), seed, tensor_id, float(std), _stream())
    return t


# ---------------------------------------------------------------- matvec


def gemv_f32(W: torch.Tensor, x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    _on_gpu(W, x)
    _need(W.dtype == torch.float32 and x.dtype == torch.float32, "gemv_f32: float32 W and x")
    M, K = W.shape
    _need(x.numel() == K, f"gemv_f32: x has {x.numel()} elements, W is {M}x{K}")
    y = torch.empty(M, dtype=torch.float32, device=W.device) if y is None else y
    call("mxd_gemv_f32", _ptr(W), _ptr(x), _ptr(y), M, K, _stream())
    return y


def matvec_f16(W, x, y=None, epilogue: str = "store", aux=None) -> torch.Tensor:
    """y (op)= W.x; W fp16 [M, K], x fp32/fp16 [K], y fp32 [M]."""
    _on_gpu(W, x)
    _need(W.dtype == torch.float16 and W.dim() == 2, "matvec_f16: W must be a 2-D float16 tensor")
    M, K = W.shape
    _need(x.numel() == K, f"matvec_f16: x has {x.numel()} elements, W is {M}x{K}")
    _need(epilogue in _EPI, f"matvec_f16: epilogue {epilogue!r}")
    if y is None:
        _need(epilogue != "add", "matvec_f16: epilogue 'add' needs y")
        y = torch.empty(M, dtype=torch.float32, device=W.device)
    _need(y.dtype == torch.float32 and y.numel() == M, "matvec_f16: y must be float32 [M]")
    if epilogue == "gelu_mul":
        _need(aux is not None and aux.numel() == M and aux.dtype == torch.float32, "matvec_f16: aux float32 [M]")
    call("mxd_matvec_f16", _ptr(W), _ptr(x), _xdtype(x), _ptr(y), M, K, _EPI[epilogue], _ptr(aux), _stream())
    return y


def matvec_f16_add(W, x, y) -> torch.Tensor:
    return matvec_f16(W, x, y, "add")


def matvec_f16_gelu_mul(W, x, aux, y=None) -> torch.Tensor:
    return matvec_f16(W, x, y, "gelu_mul", aux)


def matvec_q8b32(Wq, scales, x, y=None, epilogue: str = "store", aux=None) -> torch.Tensor:
    """y (op)= dequant(Wq, scales).x; Wq int8 [M, K], scales fp16 [M, K/32]."""
    _on_gpu(Wq, scales, x)
    _need(Wq.dtype == torch.int8 and Wq.dim() == 2, "matvec_q8b32: Wq must be a 2-D int8 tensor")
    M, K = Wq.shape
    _need(K % 32 == 0, f"matvec_q8b32: K={K} must be a multiple of 32")
    _need(scales.dtype == torch.float16 and tuple(scales.shape) == (M, K // 32), "matvec_q8b32: scales fp16 [M, K/32]")
    _need(x.numel() == K, f"matvec_q8b32: x has {x.numel()} elements, W is {M}x{K}")
    _need(epilogue in _EPI, f"matvec_q8b32: epilogue {epilogue!r}")
    if y is None:
        _need(epilogue != "add", "matvec_q8b32: epilogue 'add' needs y")
        y = torch.empty(M, dtype=torch.float32, device=Wq.device)
    if epilogue == "gelu_mul":
        _need(aux is not None and aux.numel() == M, "matvec_q8b32: aux float32 [M]")
    call(
        "mxd_matvec_q8b32", _ptr(Wq), _ptr(scales), _ptr(x), _xdtype(x), _ptr(y), M, K, _EPI[epilogue], _ptr(aux),
        _stream(),
    )
    return y


def matvec_gate_up(Wg, Wu, x, act: str = "gelu_tanh", h=None, sg=None, su=None) -> torch.Tensor:
    """h = act(Wg.x) * (Wu.x); fp16 weights, or int8 block-32 with scales sg/su."""
    _on_gpu(Wg, Wu, x)
    _need(Wg.shape == Wu.shape and Wg.dim() == 2 and Wg.dtype == Wu.dtype, "matvec_gate_up: Wg/Wu mismatch")
    F, K = Wg.shape
    _need(x.numel() == K, f"matvec_gate_up: x has {x.numel()} elements, W is {F}x{K}")
    _need(act in _ACT, f"matvec_gate_up: act {act!r}")
    if Wg.dtype == torch.float16:
        fmt = _lib.MXD_W_F16
    elif Wg.dtype == torch.int8:
        fmt = _lib.MXD_W_Q8B32
        _need(sg is not None and su is not None, "matvec_gate_up: int8 weights need sg and su")
        _need(tuple(sg.shape) == (F, K // 32) and tuple(su.shape) == (F, K // 32), "matvec_gate_up: scales shape")
    else:
        raise ValueError(f"matvec_gate_up: weight dtype {Wg.dtype}")
    h = torch.empty(F, dtype=torch.float32, device=Wg.device) if h is None else h
    call(
        "mxd_matvec_gate_up", fmt, _ptr(Wg), _ptr(sg), _ptr(Wu), _ptr(su), _ptr(x), _xdtype(x), _ptr(h), F, K,
        _ACT[act], _stream(),
    )
    return h


def matvec_gate_up_gelu(Wg, Wu, x, h=None) -> torch.Tensor:
    return matvec_gate_up(Wg, Wu, x, "gelu_tanh", h)


def matvec_gate_up_silu(Wg, Wu, x, h=None) -> torch.Tensor:
    return matvec_gate_up(Wg, Wu, x, "silu", h)


# ---------------------------------------------------------------- norms etc.


def rmsnorm(x, w, eps: float, plus_one: bool = False, y=None, out_dtype=torch.float32) -> torch.Tensor:
    """Row-wise RMSNorm of x [rows, D] (or [D])."""
    _on_gpu(x, w)
    _need(x.dtype == torch.float32 and w.dtype == torch.float32, "rmsnorm: float32 x and w")
    D = x.shape[-1]
    rows = x.numel() // D
    _need(w.numel() == D, f"rmsnorm: w has {w.numel()} elements, D={D}")
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device) if y is None else y
    call("mxd_rmsnorm", _ptr(x), _ptr(w), _ptr(y), _xdtype(y), rows, D, float(eps), int(plus_one), _stream())
    return y


def embed(E, tokens, pos: int, scale: float = 1.0, rows: int = 1, x=None) -> torch.Tensor:
    """x[r] = float(E[tokens[pos + r]]) * scale (token ids read on the device)."""
    _on_gpu(E, tokens)
    _need(E.dtype == torch.float16 and E.dim() == 2, "embed: E must be a 2-D float16 tensor")
    _need(tokens.dtype == torch.int32, "embed: tokens must be int32")
    _need(0 <= pos and pos + rows <= tokens.numel(), "embed: pos out of range")
    V, D = E.shape
    x = torch.empty((rows, D), dtype=torch.float32, device=E.device) if x is None else x
    call("mxd_embed", _ptr(E), _ptr(tokens), pos, rows, _ptr(x), D, float(scale), V, _stream())
    return x


def f32_to_f16(src, dst=None) -> torch.Tensor:
    _on_gpu(src)
    dst = torch.empty(src.shape, dtype=torch.float16, device=src.device) if dst is None else dst
    call("mxd_f32_to_f16", _ptr(src), _ptr(dst), src.numel(), _stream())
    return dst


def inv_freq(head_dim: int, theta: float) -> list[float]:
    """RoPE inverse frequencies in double, stored as float (KL/main.swift:92-94)."""
    return [1.0 / theta ** (2 * i / head_dim) for i in range(head_dim // 2)]


def tile_offsets(max_ctx: int, head_dim: int, which: str) -> np.ndarray:
    """Element offset, within one kv head's cache, of (position p, dim d) for
    the library's tiled K or V layout, as a [max_ctx, head_dim] int64 array."""
    p = np.arange(max_ctx)[:, None]
    d = np.arange(head_dim)[None, :]
    k = p & 31
    base = (p & ~31) * head_dim
    if which == "k":
        t, col = (k >> 2) & 1, ((k >> 3) << 2) | (k & 3)
        c, g, e = d >> 5, (d >> 3) & 3, d & 7
        return base + ((t * (head_dim >> 5) + c) * 64 + g * 16 + col) * 8 + e
    if which == "v":
        return base + ((d >> 4) * 64 + (k >> 3) * 16 + (d & 15)) * 8 + (k & 7)
    raise ValueError(which)


def to_tiles(rows, which: str):
    """Cache rows [n_kv, max_ctx, hd] (the reference's layout) -> the library's
    tiled K ("k") or V ("v") storage, same shape; numpy arrays or torch tensors."""
    n_kv, ctx, hd = rows.shape
    off = tile_offsets(ctx, hd, which).reshape(-1)
    if isinstance(rows, torch.Tensor):
        out = torch.empty_like(rows).reshape(n_kv, -1)
        out[:, torch.from_numpy(off).to(rows.device)] = rows.reshape(n_kv, -1)
        return out.reshape(n_kv, ctx, hd)
    out = np.empty_like(rows).reshape(n_kv, -1)
    out[:, off] = rows.reshape(n_kv, -1)
    return out.reshape(n_kv, ctx, hd)


def from_tiles(tiles, which: str):
    """Inverse of to_tiles."""
    n_kv, ctx, hd = tiles.shape
    off = tile_offsets(ctx, hd, which).reshape(-1)
    if isinstance(tiles, torch.Tensor):
        return tiles.reshape(n_kv, -1)[:, torch.from_numpy(off).to(tiles.device)].reshape(n_kv, ctx, hd)
    return tiles.reshape(n_kv, -1)[:, off].reshape(n_kv, ctx, hd)


def _check_caches(kcache, vcache, fn: str):
    n_kv, max_ctx, hd = kcache.shape
    _need(max_ctx % 32 == 0, f"{fn}: max_ctx={max_ctx} must be a multiple of 32")
    _need(tuple(vcache.shape) == (n_kv, max_ctx, hd), f"{fn}: kcache and vcache must both be [n_kv, max_ctx, hd]")
    _need(kcache.dtype == torch.float16 and vcache.dtype == torch.float16, f"{fn}: fp16 caches")
    return n_kv, max_ctx, hd


def rope_kv(qkv, kcache, vcache, inv_freq_t, n_heads: int, n_kv_heads: int, pos0: int) -> None:
    """Rotate q in place and k, append k and v (fp16) to the caches at pos0 + row.
    kcache, vcache: [n_kv, max_ctx, hd] fp16 in the tiled layout (to_tiles)."""
    _on_gpu(qkv, kcache, vcache, inv_freq_t)
    n_kv, max_ctx, hd = _check_caches(kcache, vcache, "rope_kv")
    _need(n_kv == n_kv_heads, "rope_kv: cache has a different number of kv heads")
    row_len = (n_heads + 2 * n_kv_heads) * hd
    _need(qkv.dtype == torch.float32 and qkv.numel() % row_len == 0, f"rope_kv: qkv rows of {row_len} floats")
    rows = qkv.numel() // row_len
    _need(inv_freq_t.numel() == hd // 2, "rope_kv: inv_freq has head_dim/2 entries")
    call(
        "mxd_rope_kv", _ptr(qkv), _ptr(kcache), _ptr(vcache), _ptr(inv_freq_t), n_heads, n_kv_heads, hd, max_ctx,
        pos0, rows, _stream(),
    )


def attention_workspace(n_heads: int, n_kv_heads: int, head_dim: int, max_ctx: int, device="cuda") -> torch.Tensor:
    """Zeroed once here; the kernel leaves its counters at zero after every call."""
    nbytes = query("mxd_attention_workspace_size", n_heads, n_kv_heads, head_dim, max_ctx)
    return torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=device)


def attention(q, kcache, vcache, n_keys: int, n_heads: int, scale: float | None = None, out=None, workspace=None,
              pos_dev=None, window: int = 0) -> torch.Tensor:
    """Single-query attention of q [n_heads*hd] over keys [0, n_keys) of the
    tiled caches (kcache, vcache [n_kv, max_ctx, hd], see to_tiles); with a
    window, over the last `window` of them (a Gemma-4 sliding layer)."""
    _on_gpu(q, kcache, vcache)
    n_kv, max_ctx, hd = _check_caches(kcache, vcache, "attention")
    _need(q.numel() == n_heads * hd and q.dtype == torch.float32, "attention: q float32 [n_heads*hd]")
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    out = torch.empty(n_heads * hd, dtype=torch.float32, device=q.device) if out is None else out
    if workspace is None:
        workspace = attention_workspace(n_heads, n_kv, hd, max_ctx, q.device)
    if window:
        call(
            "mxd_attention_window", _ptr(q), _ptr(kcache), _ptr(vcache), _ptr(out), n_heads, n_kv, hd, max_ctx,
            int(n_keys), _ptr(pos_dev), int(window), float(scale), _ptr(workspace), workspace.numel(), _stream(),
        )
        return out
    call(
        "mxd_attention", _ptr(q), _ptr(kcache), _ptr(vcache), _ptr(out), n_heads, n_kv, hd, max_ctx, int(n_keys),
        _ptr(pos_dev), float(scale), _ptr(workspace), workspace.numel(), _stream(),
    )
    return out


def attention_split(q, kcache, vcache, n_keys: int, n_heads: int, n_splits: int, scale: float | None = None,
                    partials=None, pos_dev=None, window: int = 0) -> torch.Tensor:
    """The split half of attention without its merge: a float32 buffer of
    n_splits unnormalised partials, O [n_splits, n_heads, hd] then (max, sum)
    [n_splits, n_heads, 2] (log2-domain scores), for matvec_f16_attn_merge."""
    _on_gpu(q, kcache, vcache)
    n_kv, max_ctx, hd = _check_caches(kcache, vcache, "attention_split")
    _need(q.numel() == n_heads * hd and q.dtype == torch.float32, "attention_split: q float32 [n_heads*hd]")
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    n = n_splits * n_heads * (hd + 2)
    partials = torch.empty(n, dtype=torch.float32, device=q.device) if partials is None else partials
    _need(partials.dtype == torch.float32 and partials.numel() >= n, f"attention_split: partials float32 [{n}]")
    call(
        "mxd_attention_split_window", _ptr(q), _ptr(kcache), _ptr(vcache), n_heads, n_kv, hd, max_ctx, int(n_keys),
        _ptr(pos_dev), int(window), float(scale), int(n_splits), _ptr(partials), partials.numel() * 4, _stream(),
    )
    return partials


def matvec_f16_attn_merge(W, partials, n_splits: int, n_heads: int, head_dim: int, max_ctx: int, n_keys: int,
                          y=None, epilogue: str = "store", pos_dev=None, window: int = 0) -> torch.Tensor:
    """y (op)= W . x with x the log-sum-exp merge of attention_split's partials."""
    _on_gpu(W, partials)
    M, K = W.shape
    _need(W.dtype == torch.float16 and K == n_heads * head_dim, "matvec_f16_attn_merge: W fp16 [M, n_heads*hd]")
    _need(partials.dtype == torch.float32, "matvec_f16_attn_merge: partials float32")
    if y is None:
        _need(epilogue == "store", "matvec_f16_attn_merge: epilogue 'add' needs y")
        y = torch.empty(M, dtype=torch.float32, device=W.device)
    call(
        "mxd_matvec_f16_attn_merge_window", _ptr(W), _ptr(partials), int(n_splits), n_heads, head_dim, max_ctx,
        int(n_keys), _ptr(pos_dev), int(window), _ptr(y), M, _EPI[epilogue], None, _stream(),
    )
    return y


def attention_prefill(q, kcache, vcache, pos0: int, n_heads: int, scale: float | None = None, out=None,
                      q_stride: int | None = None, rows: int | None = None, window: int = 0) -> torch.Tensor:
    """Causal attention of a prefill chunk: row t of q (rows q_stride floats
    apart; the q part of a qkv row [rows, qkv_dim] works in place) is the query
    at position pos0 + t over keys [0, pos0 + t] of the tiled caches (with a
    window, the last `window` of them). Returns out [rows, n_heads * hd]."""
    _on_gpu(q, kcache, vcache)
    n_kv, max_ctx, hd = _check_caches(kcache, vcache, "attention_prefill")
    _need(q.dtype == torch.float32 and q.is_contiguous() and q.dim() == 2, "attention_prefill: q float32 [rows, stride]")
    rows = q.shape[0] if rows is None else rows
    q_stride = q.shape[1] if q_stride is None else q_stride
    _need(q.numel() >= (rows - 1) * q_stride + n_heads * hd, "attention_prefill: q too small for rows x stride")
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    out = torch.empty((rows, n_heads * hd), dtype=torch.float32, device=q.device) if out is None else out
    _need(out.dtype == torch.float32 and out.is_contiguous() and out.numel() == rows * n_heads * hd,
          "attention_prefill: out float32 [rows, n_heads * hd]")
    if window:
        call("mxd_attention_prefill_window", _ptr(q), q_stride, _ptr(kcache), _ptr(vcache), _ptr(out), n_heads * hd,
             n_heads, n_kv, hd, max_ctx, int(pos0), int(rows), int(window), float(scale), _stream())
        return out
    call("mxd_attention_prefill", _ptr(q), q_stride, _ptr(kcache), _ptr(vcache), _ptr(out), n_heads * hd, n_heads,
         n_kv, hd, max_ctx, int(pos0), int(rows), float(scale), _stream())
    return out


# ---------------------------------------------------------------- Gemma-4


def rmsnorm_add(src, w, x, eps: float, post: float = 1.0) -> torch.Tensor:
    """x = (x + rmsnorm(src) * w) * post per row (src, x float32 [rows, D] or [D])."""
    _on_gpu(src, w, x)
    D = w.numel()
    _need(src.dtype == torch.float32 and x.dtype == torch.float32 and w.dtype == torch.float32,
          "rmsnorm_add: float32 tensors")
    _need(src.numel() == x.numel() and x.numel() % D == 0, "rmsnorm_add: src and x are rows of len(w)")
    call("mxd_rmsnorm_add", _ptr(src), _ptr(w), _ptr(x), x.numel() // D, D, float(eps), float(post), _stream())
    return x


def matvec_f16_residual(W, x, res_src, res_w, x_out, eps: float, res_post: float = 1.0, norm_w=None, y=None,
                        epilogue: str = "store", aux=None) -> torch.Tensor:
    """x_out = (x + rmsnorm(res_src) * res_w) * res_post, then y (op)= W . x_out
    (W . rmsnorm(x_out) * norm_w with norm_w), in one launch."""
    _on_gpu(W, x, res_src, res_w, x_out)
    M, K = W.shape
    _need(W.dtype == torch.float16 and x.dtype == torch.float32 and x.numel() == K,
          "matvec_f16_residual: W fp16 [M, K], x float32 [K]")
    _need(res_src.numel() == K and res_w.numel() == K and x_out.numel() == K, "matvec_f16_residual: vectors of K")
    if y is None:
        _need(epilogue != "add", "matvec_f16_residual: epilogue 'add' needs y")
        y = torch.empty(M, dtype=torch.float32, device=W.device)
    call("mxd_matvec_f16_residual", _ptr(W), _ptr(x), _ptr(res_src), _ptr(res_w), float(res_post), _ptr(x_out),
         _ptr(norm_w), float(eps), 0, _ptr(y), M, K, _EPI[epilogue], _ptr(aux), _stream())
    return y


def gate_up_residual(Wg, Wu, x, res_src, res_w, x_out, norm_w, eps: float, res_post: float = 1.0,
                     act: str = "gelu_tanh", h=None) -> torch.Tensor:
    """x_out = (x + rmsnorm(res_src) * res_w) * res_post, then
    h = act(Wg . n) * (Wu . n) with n = rmsnorm(x_out) * norm_w, in one launch."""
    _on_gpu(Wg, Wu, x, res_src, res_w, x_out, norm_w)
    F, K = Wg.shape
    _need(Wu.shape == Wg.shape and Wg.dtype == torch.float16, "gate_up_residual: Wg, Wu fp16 [F, K]")
    h = torch.empty(F, dtype=torch.float32, device=Wg.device) if h is None else h
    call("mxd_gate_up_residual", _ptr(Wg), _ptr(Wu), _ptr(x), _ptr(res_src), _ptr(res_w), float(res_post), _ptr(x_out),
         _ptr(norm_w), float(eps), 0, _ptr(h), F, K, _ACT[act], _stream())
    return h


def ple_combine(proj, ple, w, n_layers: int, dim: int, eps: float) -> torch.Tensor:
    """ple = (rmsnorm(proj / sqrt(dim)) * w + ple) / sqrt(2) over each of the
    n_layers slices of len(w) values per row (proj, ple float32 [rows, n_layers * P])."""
    _on_gpu(proj, ple, w)
    P = w.numel()
    _need(proj.dtype == ple.dtype == w.dtype == torch.float32, "ple_combine: float32 tensors")
    _need(proj.numel() == ple.numel() and ple.numel() % (n_layers * P) == 0,
          "ple_combine: proj and ple are rows of n_layers * len(w)")
    rows = ple.numel() // (n_layers * P)
    call("mxd_ple_combine", _ptr(proj), _ptr(ple), _ptr(w), rows, n_layers, P, 1.0 / math.sqrt(dim), float(eps),
         _stream())
    return ple


def qk_norm_rope_kv(qkv, kcache, vcache, q_w, k_w, inv_freq_t, n_heads: int, rope_pairs: int, eps: float,
                    pos0: int = 0, pos_dev=None, head_dim: int | None = None) -> None:
    """Per-head RMSNorm of q (q_w), k (k_w), v (no weight), RoPE over the first
    rope_pairs pairs of q and k, q back in place, k and v appended (fp16) at
    pos0 + row. kcache None: q only (a layer sharing another's cache; give
    head_dim)."""
    _on_gpu(qkv, q_w, inv_freq_t)
    if kcache is not None:
        _on_gpu(kcache, vcache, k_w)
        n_kv, max_ctx, hd = _check_caches(kcache, vcache, "qk_norm_rope_kv")
    else:
        _need(head_dim is not None, "qk_norm_rope_kv: head_dim is needed without caches")
        n_kv, max_ctx, hd = 0, 32, head_dim
    row_len = (n_heads + 2 * n_kv) * hd
    _need(qkv.dtype == torch.float32 and qkv.numel() % row_len == 0, f"qk_norm_rope_kv: qkv rows of {row_len} floats")
    _need(q_w.numel() == hd and (k_w is None or k_w.numel() == hd), "qk_norm_rope_kv: norm weights of head_dim")
    _need(inv_freq_t.numel() >= hd // 2, "qk_norm_rope_kv: inv_freq has head_dim/2 entries")
    call("mxd_qk_norm_rope_kv", _ptr(qkv), _ptr(kcache), _ptr(vcache), _ptr(q_w), _ptr(k_w), _ptr(inv_freq_t),
         n_heads, n_kv, hd, int(rope_pairs), max_ctx, float(eps), int(pos0), qkv.numel() // row_len, _ptr(pos_dev),
         _stream())


def gemm_workspace(n_rows: int, M: int, K: int, glu: bool = False, device="cuda") -> torch.Tensor:
    name = "mxd_gemm_gate_up_f16_workspace_size" if glu else "mxd_gemm_f16_workspace_size"
    return torch.empty(max(query(name, n_rows, M, K), 16), dtype=torch.uint8, device=device)


def gemm_f16(W, X, Y=None, epilogue: str = "store", workspace=None) -> torch.Tensor:
    """Y[b] (op)= W . X[b]: fp16 W [M, K], X fp16 or fp32 [B, K] (fp32 is
    rounded to fp16 as it is loaded), Y fp32 [B, M] (gemm_f16 / gemm_f16_add
    of the reference's prefill)."""
    _on_gpu(W, X)
    M, K = W.shape
    _need(W.dtype == torch.float16 and W.is_contiguous(), "gemm_f16: W float16 [M, K]")
    _need(X.dtype in (torch.float16, torch.float32) and X.dim() == 2 and X.shape[1] == K and X.is_contiguous(),
          "gemm_f16: X float16 or float32 [B, K]")
    B = X.shape[0]
    if Y is None:
        _need(epilogue == "store", "gemm_f16: epilogue 'add' needs Y")
        Y = torch.empty((B, M), dtype=torch.float32, device=X.device)
    _need(Y.is_contiguous() and Y.dtype == torch.float32 and Y.numel() == B * M, "gemm_f16: Y float32 [B, M]")
    if workspace is None:
        workspace = gemm_workspace(B, M, K, False, X.device)
    call("mxd_gemm_f16", _ptr(W), _ptr(X), _xdtype(X), _ptr(Y), B, M, K, _EPI[epilogue], _ptr(workspace),
         workspace.numel(), _stream())
    return Y


def gemm_f16_add(W, X, Y, workspace=None) -> torch.Tensor:
    return gemm_f16(W, X, Y, "add", workspace)


def gemm_gate_up(Wg, Wu, X, act: str = "gelu_tanh", H=None, workspace=None) -> torch.Tensor:
    """H[b] = act(Wg . X[b]) * (Wu . X[b]): fp16 Wg, Wu [F, K], X fp16 [B, K],
    H fp32 [B, F] (gemm_gate_up_silu of the reference's prefill, and GeGLU)."""
    _on_gpu(Wg, Wu, X)
    F, K = Wg.shape
    _need(Wg.dtype == torch.float16 and Wu.dtype == torch.float16 and tuple(Wu.shape) == (F, K),
          "gemm_gate_up: Wg, Wu float16 [F, K]")
    _need(X.dtype == torch.float16 and X.dim() == 2 and X.shape[1] == K and X.is_contiguous(),
          "gemm_gate_up: X float16 [B, K]")
    B = X.shape[0]
    H = torch.empty((B, F), dtype=torch.float32, device=X.device) if H is None else H
    _need(H.is_contiguous() and H.dtype == torch.float32 and H.numel() == B * F, "gemm_gate_up: H float32 [B, F]")
    if workspace is None:
        workspace = gemm_workspace(B, F, K, True, X.device)
    call("mxd_gemm_gate_up_f16", _ptr(Wg), _ptr(Wu), _ptr(X), _ptr(H), B, F, K, _ACT[act], _ptr(workspace),
         workspace.numel(), _stream())
    return H


def argmax_workspace(device="cuda") -> torch.Tensor:
    """Zeroed once here; the kernel leaves it zeroed after every call."""
    return torch.zeros(max(query("mxd_argmax_workspace_size", 0), 16), dtype=torch.uint8, device=device)


def argmax(logits, tokens, out_idx: int, workspace) -> None:
    """tokens[out_idx] = argmax(logits), ties to the lowest index."""
    _on_gpu(logits, tokens)
    _need(logits.dtype == torch.float32 and tokens.dtype == torch.int32, "argmax: float32 logits, int32 tokens")
    _need(0 <= out_idx < tokens.numel(), "argmax: out_idx out of range")
    call("mxd_argmax", _ptr(logits), _ptr(tokens), logits.numel(), out_idx, _ptr(workspace), workspace.numel(), _stream())
