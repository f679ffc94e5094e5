"""Ragged-batch decode over a paged KV cache.

The reference decodes one sequence at a time over a contiguous cache and has
no paging or batching (ios_kernels/surfaces/DESIGN_AND_LIMITATIONS.md:48,87-88).
Here a batch of B sequences of different lengths decodes one token each per
step, in one launch per operator:

    pack_ragged          page tables for a set of sequence lengths (16-key pages,
                         physical pages in any order)
    PagedCache           per-layer page pools + page table + host-side fill/read
    rope_kv_paged        RoPE + KV append of every sequence at its own position
    attention_paged      split-L GQA attention of every sequence over its pages
    gemm_q8b32           Y (+)= X . W^T, int8 block-32 W, X fp16 [B, K] (matrix
                         cores from 16 rows on, one matvec per row below)
    gemm_gate_up_q8b32   H = act(X . Wg^T) * (X . Wu^T)
    RaggedLayerQ8        one Llama-shaped layer (int8 weights) stepping a batch

Row b of every activation matrix belongs to sequence b; seq_lens[b] counts the
keys of sequence b after this step's append. Page layout (slab offsets) as in
include/mxdecode.h.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib, ops
from ._lib import call, query
from .quant import quantize_q8b32

PAGE = 16


def page_offsets(head_dim: int, which: str) -> np.ndarray:
    """Offset (in halfs) of (key r, dim d) inside a (page, kv head) slab, as a
    [16, head_dim] int64 array: the slab holds one half of a 32-position tile
    of the contiguous layout, each MFMA operand piece contiguous."""
    r = np.arange(PAGE)[:, None]
    d = np.arange(head_dim)[None, :]
    if which == "k":
        rr = ((r >> 3) << 2) | (r & 3)
        return ((((d >> 5) * 2 + ((r >> 2) & 1)) * 4 + ((d >> 3) & 3)) * 8 + rr) * 8 + (d & 7)
    if which == "v":
        return (((d >> 4) * 2 + (r >> 3)) * 16 + (d & 15)) * 8 + (r & 7)
    raise ValueError(which)


def pack_ragged(seq_lens, seed: int | None = None, spare_pages: int = 0) -> tuple[np.ndarray, int]:
    """Page table (int32 [B, max_pages], -1 where unused) giving every sequence
    ceil(len / 16) pages of one shared pool, and the pool size. With a seed the
    physical pages are a random permutation of the pool (pages of a sequence
    are not contiguous), otherwise they are dealt in order."""
    lens = np.asarray(seq_lens, dtype=np.int64)
    _need((lens >= 0).all(), "pack_ragged: negative length")
    need = (lens + PAGE - 1) // PAGE
    max_pages = max(1, int(need.max()) if len(need) else 1)
    n_pages = int(need.sum()) + spare_pages
    ids = np.arange(n_pages, dtype=np.int32)
    if seed is not None:
        ids = np.random.default_rng(seed).permutation(n_pages).astype(np.int32)
    table = np.full((len(lens), max_pages), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        table[b, :n] = ids[at : at + n]
        at += n
    return table, max(n_pages, 1)


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


class PagedCache:
    """K and V page pools of n_layers layers: [n_layers, n_pages, n_kv, 16, hd]
    fp16 each (a (page, kv head) slab is 16 * hd contiguous halfs in the MFMA
    order of page_offsets), plus the page table on the device."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, page_table: np.ndarray, n_pages: int,
                 device="cuda"):
        self.n_layers, self.n_kv, self.hd = n_layers, n_kv_heads, head_dim
        self.n_pages = n_pages
        self.table_host = np.ascontiguousarray(page_table, dtype=np.int32)
        self.max_pages = self.table_host.shape[1]
        shape = (n_layers, n_pages, n_kv_heads, PAGE, head_dim)
        self.k = torch.zeros(shape, dtype=torch.float16, device=device)
        self.v = torch.zeros(shape, dtype=torch.float16, device=device)
        self.table = torch.from_numpy(self.table_host).to(device)
        self._off = {w: page_offsets(head_dim, w) for w in ("k", "v")}

    def _index(self, b: int, n: int, which: str) -> np.ndarray:
        """Flat indices (within one layer's pool) of positions 0..n-1 of
        sequence b, shaped [n_kv, n, hd]."""
        p = np.arange(n)
        pages = self.table_host[b, p // PAGE].astype(np.int64)
        _need((pages >= 0).all() and (pages < self.n_pages).all(), "PagedCache: position without a page")
        slab = PAGE * self.hd
        base = pages[None, :, None] * (self.n_kv * slab) + np.arange(self.n_kv)[:, None, None] * slab
        return base + self._off[which][p % PAGE][None, :, :]

    def write(self, layer: int, b: int, k_rows, v_rows) -> None:
        """Store positions 0..n-1 of sequence b from reference-layout rows
        [n_kv, n, hd] (numpy or torch)."""
        for which, rows, pool in (("k", k_rows, self.k), ("v", v_rows, self.v)):
            rows = torch.as_tensor(rows, dtype=torch.float16).to(pool.device)
            _need(rows.shape[0] == self.n_kv and rows.shape[2] == self.hd, "PagedCache.write: rows [n_kv, n, hd]")
            idx = torch.from_numpy(self._index(b, rows.shape[1], which)).to(pool.device)
            pool[layer].view(-1)[idx.reshape(-1)] = rows.reshape(-1)

    def read(self, layer: int, b: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        """Positions 0..n-1 of sequence b as reference-layout rows [n_kv, n, hd]."""
        out = []
        for which, pool in (("k", self.k), ("v", self.v)):
            idx = torch.from_numpy(self._index(b, n, which)).to(pool.device)
            out.append(pool[layer].view(-1)[idx.reshape(-1)].reshape(self.n_kv, n, self.hd).cpu().numpy())
        return out[0], out[1]


# ---------------------------------------------------------------- operators


def rope_kv_paged(qkv, kpool, vpool, inv_freq_t, n_heads: int, n_kv_heads: int, page_table, seq_lens) -> None:
    """Rotate q and k of every row of qkv [B, (NH + 2 NKV) hd] in place at
    position seq_lens[b] - 1 and append k, v to that position's page.
    kpool / vpool: one layer's pools [n_pages, n_kv, 16, hd] fp16."""
    ops._on_gpu(qkv, kpool, vpool, inv_freq_t, page_table, seq_lens)
    n_pages, n_kv, page, hd = kpool.shape
    _need(page == PAGE and n_kv == n_kv_heads and tuple(vpool.shape) == tuple(kpool.shape),
          "rope_kv_paged: pools [n_pages, n_kv, 16, hd]")
    B = seq_lens.numel()
    _need(qkv.dtype == torch.float32 and qkv.numel() == B * (n_heads + 2 * n_kv_heads) * hd,
          "rope_kv_paged: qkv float32 [B, (n_heads + 2 n_kv_heads) head_dim]")
    _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.shape[0] == B,
          "rope_kv_paged: page_table int32 [B, max_pages]")
    call("mxd_rope_kv_paged", qkv.data_ptr(), kpool.data_ptr(), vpool.data_ptr(), n_pages, inv_freq_t.data_ptr(),
         n_heads, n_kv_heads, hd, page_table.data_ptr(), page_table.shape[1], seq_lens.data_ptr(), B, ops._stream())


def attention_paged_workspace(n_heads: int, n_kv_heads: int, head_dim: int, n_seqs: int, max_keys: int,
                              device="cuda") -> torch.Tensor:
    nbytes = query("mxd_attention_paged_workspace_size", n_heads, n_kv_heads, head_dim, n_seqs, max_keys)
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def attention_paged(q, kpool, vpool, page_table, seq_lens, n_heads: int, max_keys: int, q_stride: int | None = None,
                    out=None, scale: float | None = None, workspace=None) -> torch.Tensor:
    """out[b] = attention of q row b over the seq_lens[b] keys of sequence b.
    q: float32 with B rows q_stride floats apart (the q part of qkv rows works
    in place); out float32 [B, n_heads * hd]."""
    ops._on_gpu(kpool, vpool, page_table, seq_lens)
    _need(q.is_cuda and q.dtype == torch.float32, "attention_paged: q float32 on the GPU")
    n_pages, n_kv, page, hd = kpool.shape
    _need(page == PAGE and tuple(vpool.shape) == tuple(kpool.shape), "attention_paged: pools [n_pages, n_kv, 16, hd]")
    B = seq_lens.numel()
    q_stride = n_heads * hd if q_stride is None else q_stride
    _need(q.is_contiguous() and q.numel() >= (B - 1) * q_stride + n_heads * hd, "attention_paged: q too small")
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    out = torch.empty((B, n_heads * hd), dtype=torch.float32, device=q.device) if out is None else out
    _need(out.is_contiguous() and out.numel() == B * n_heads * hd, "attention_paged: out float32 [B, n_heads*hd]")
    if workspace is None:
        workspace = attention_paged_workspace(n_heads, n_kv, hd, B, max_keys, q.device)
    call("mxd_attention_paged", q.data_ptr(), q_stride, kpool.data_ptr(), vpool.data_ptr(), n_pages,
         page_table.data_ptr(), page_table.shape[1], seq_lens.data_ptr(), B, out.data_ptr(), n_heads * hd, n_heads,
         n_kv, hd, int(max_keys), float(scale), workspace.data_ptr(), workspace.numel(), ops._stream())
    return out


def gemm_workspace(n_rows: int, M: int, K: int, glu: bool = False, device="cuda") -> torch.Tensor:
    name = "mxd_gemm_gate_up_q8b32_workspace_size" if glu else "mxd_gemm_q8b32_workspace_size"
    return torch.empty(max(query(name, n_rows, M, K), 16), dtype=torch.uint8, device=device)


def gemm_q8b32(Wq, scales, X, Y=None, epilogue: str = "store", workspace=None) -> torch.Tensor:
    """Y[b] (op)= dequant(Wq, scales) . X[b]; X fp16 or fp32 [B, K] (fp32 is
    rounded to fp16 as it is loaded), Y fp32 [B, M]."""
    ops._on_gpu(Wq, scales, X)
    M, K = Wq.shape
    _need(Wq.dtype == torch.int8 and scales.dtype == torch.float16 and tuple(scales.shape) == (M, K // 32),
          "gemm_q8b32: int8 Wq [M, K] and fp16 scales [M, K/32]")
    _need(X.dtype in (torch.float16, torch.float32) and X.dim() == 2 and X.shape[1] == K and X.is_contiguous(),
          "gemm_q8b32: X fp16 or fp32 [B, K]")
    B = X.shape[0]
    if Y is None:
        _need(epilogue == "store", "gemm_q8b32: epilogue 'add' needs Y")
        Y = torch.empty((B, M), dtype=torch.float32, device=X.device)
    _need(Y.is_contiguous() and Y.dtype == torch.float32 and Y.numel() == B * M, "gemm_q8b32: Y fp32 [B, M]")
    if workspace is None:
        workspace = gemm_workspace(B, M, K, False, X.device)
    call("mxd_gemm_q8b32", Wq.data_ptr(), scales.data_ptr(), X.data_ptr(), ops._xdtype(X), Y.data_ptr(), B, M, K,
         ops._EPI[epilogue], workspace.data_ptr(), workspace.numel(), ops._stream())
    return Y


def gemm_q8b32_partials_bytes(n_rows: int, M: int, K: int) -> int:
    """Bytes gemm_q8b32_partials leaves for these sizes (0: not a matrix-core product)."""
    return query("mxd_gemm_q8b32_partials_size", n_rows, M, K)


def gemm_q8b32_partials(Wq, scales, X, part) -> int:
    """The K-split partial products of gemm_q8b32 (store) left unsummed in
    part (fp32, at least gemm_q8b32_partials_bytes); returns their count.
    rope_kv_paged_sum and rmsnorm_residual_sum add them as they load them.
    Needs B >= 16 and K % 128 == 0."""
    ops._on_gpu(Wq, scales, X, part)
    M, K = Wq.shape
    _need(Wq.dtype == torch.int8 and scales.dtype == torch.float16 and tuple(scales.shape) == (M, K // 32),
          "gemm_q8b32_partials: int8 Wq [M, K] and fp16 scales [M, K/32]")
    _need(X.dtype in (torch.float16, torch.float32) and X.dim() == 2 and X.shape[1] == K and X.is_contiguous(),
          "gemm_q8b32_partials: X fp16 or fp32 [B, K]")
    _need(part.is_contiguous() and part.dtype == torch.float32, "gemm_q8b32_partials: part fp32")
    n = ctypes.c_int(0)
    call("mxd_gemm_q8b32_partials", Wq.data_ptr(), scales.data_ptr(), X.data_ptr(), ops._xdtype(X), part.data_ptr(),
         part.numel() * 4, X.shape[0], M, K, ctypes.byref(n), ops._stream())
    return n.value


def rope_kv_paged_sum(part, n_splits: int, qkv, kpool, vpool, inv_freq_t, n_heads: int, n_kv_heads: int, page_table,
                      seq_lens) -> None:
    """rope_kv_paged over the sum of n_splits partials of the q|k|v product
    (part as gemm_q8b32_partials leaves it): the rotated q goes to qkv, k and v
    to the pages."""
    ops._on_gpu(part, qkv, kpool, vpool, inv_freq_t, page_table, seq_lens)
    n_pages, n_kv, page, hd = kpool.shape
    _need(page == PAGE and n_kv == n_kv_heads and tuple(vpool.shape) == tuple(kpool.shape),
          "rope_kv_paged_sum: pools [n_pages, n_kv, 16, hd]")
    B = seq_lens.numel()
    row = (n_heads + 2 * n_kv_heads) * hd
    _need(qkv.dtype == torch.float32 and qkv.numel() == B * row, "rope_kv_paged_sum: qkv float32 [B, (NH + 2 NKV) hd]")
    _need(part.dtype == torch.float32 and part.numel() >= n_splits * B * row, "rope_kv_paged_sum: part too small")
    _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.shape[0] == B,
          "rope_kv_paged_sum: page_table int32 [B, max_pages]")
    call("mxd_rope_kv_paged_sum", part.data_ptr(), n_splits, qkv.data_ptr(), kpool.data_ptr(), vpool.data_ptr(),
         n_pages, inv_freq_t.data_ptr(), n_heads, n_kv_heads, hd, page_table.data_ptr(), page_table.shape[1],
         seq_lens.data_ptr(), B, ops._stream())


def rmsnorm_residual_sum(X, part, n_splits: int, w, eps: float, plus_one: bool, y) -> None:
    """X += the sum of n_splits partials of a product with X's shape (part as
    gemm_q8b32_partials leaves it), then y = rmsnorm(X) (fp16 or fp32 y)."""
    ops._on_gpu(X, part, w, y)
    B, D = X.shape
    _need(X.dtype == torch.float32 and X.is_contiguous(), "rmsnorm_residual_sum: X fp32 [B, D]")
    _need(part.dtype == torch.float32 and part.numel() >= n_splits * B * D, "rmsnorm_residual_sum: part too small")
    _need(y.is_contiguous() and y.numel() == B * D and y.dtype in (torch.float16, torch.float32),
          "rmsnorm_residual_sum: y fp16 or fp32 [B, D]")
    call("mxd_rmsnorm_residual_sum", X.data_ptr(), part.data_ptr(), n_splits, w.data_ptr(), y.data_ptr(),
         _lib.MXD_F16 if y.dtype == torch.float16 else _lib.MXD_F32, B, D, float(eps), int(plus_one), ops._stream())


def gemm_gate_up_q8b32(Wg, sg, Wu, su, X, act: str = "silu", H=None, workspace=None) -> torch.Tensor:
    """H[b] = act(Wg . X[b]) * (Wu . X[b]); X fp16 [B, K], H fp32 [B, F]."""
    ops._on_gpu(Wg, sg, Wu, su, X)
    F, K = Wg.shape
    _need(tuple(Wu.shape) == (F, K), "gemm_gate_up_q8b32: Wg and Wu must have the same shape")
    _need(X.dtype == torch.float16 and X.dim() == 2 and X.shape[1] == K, "gemm_gate_up_q8b32: X fp16 [B, K]")
    B = X.shape[0]
    H = torch.empty((B, F), dtype=torch.float32, device=X.device) if H is None else H
    _need(H.is_contiguous() and H.dtype == torch.float32 and H.numel() == B * F, "gemm_gate_up_q8b32: H fp32 [B, F]")
    if workspace is None:
        workspace = gemm_workspace(B, F, K, True, X.device)
    call("mxd_gemm_gate_up_q8b32", Wg.data_ptr(), sg.data_ptr(), Wu.data_ptr(), su.data_ptr(), X.data_ptr(),
         H.data_ptr(), B, F, K, ops._ACT[act], workspace.data_ptr(), workspace.numel(), ops._stream())
    return H


# ---------------------------------------------------------------- the layer


@dataclass(frozen=True)
class LayerShape:
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    eps: float = 1e-5
    rope_theta: float = 10000.0
    act: str = "silu"
    plus_one: bool = False

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    @property
    def weight_bytes(self) -> int:
        """int8 weights + fp16 block scales + fp32 norms."""
        D, F = self.dim, self.ffn_dim
        mats = self.qkv_dim * D + D * self.n_heads * self.head_dim + 2 * F * D + D * F
        return mats + mats // 16 + 2 * D * 4


LLAMA3_8B_LAYER = LayerShape(dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=14336)

WEIGHTS = ("wqkv", "wo", "wgate", "wup", "wdown")


class RaggedLayerQ8:
    """One Llama-shaped layer with int8 block-32 weights that steps a ragged
    batch: rmsnorm -> qkv -> rope_kv_paged -> attention_paged -> o (+x) ->
    rmsnorm -> gate/up (SwiGLU) -> down (+x), the reference's per-layer order
    (KL/main.swift:321-347). Workspaces and activations are allocated once
    for batches of up to max_batch rows; step() allocates nothing.

    From 16 rows on (fold_sums, the default) the qkv and o products leave
    their K-split partials unsummed and the next op adds them as it loads
    them (rope_kv_paged_sum, rmsnorm_residual_sum): two launches fewer per
    step, with results bit-identical to the summing products."""

    def __init__(self, shape: LayerShape, weights: dict, max_batch: int, max_keys: int, device="cuda",
                 fold_sums: bool = True):
        self.s, self.dev, self.max_keys = shape, torch.device(device), max_keys
        s = shape
        D, F, QD = s.dim, s.ffn_dim, s.n_heads * s.head_dim
        self.W = {}
        for name in WEIGHTS:
            q, sc = weights[name]
            self.W[name] = (torch.as_tensor(q).to(self.dev).contiguous(),
                            torch.as_tensor(sc).to(self.dev).contiguous())
        self.attn_norm = torch.as_tensor(weights["attn_norm"], dtype=torch.float32).to(self.dev)
        self.ffn_norm = torch.as_tensor(weights["ffn_norm"], dtype=torch.float32).to(self.dev)
        self.invf = torch.tensor(ops.inv_freq(s.head_dim, s.rope_theta), dtype=torch.float32, device=self.dev)
        B = max_batch
        self.xn = torch.empty((B, D), dtype=torch.float16, device=self.dev)
        self.qkv = torch.empty((B, s.qkv_dim), dtype=torch.float32, device=self.dev)
        self.att = torch.empty((B, QD), dtype=torch.float32, device=self.dev)
        self.h = torch.empty((B, F), dtype=torch.float32, device=self.dev)
        self.ws = {
            "wqkv": gemm_workspace(B, s.qkv_dim, D, False, self.dev),
            "wo": gemm_workspace(B, D, QD, False, self.dev),
            "glu": gemm_workspace(B, F, D, True, self.dev),
            "wdown": gemm_workspace(B, D, F, False, self.dev),
            "attn": attention_paged_workspace(s.n_heads, s.n_kv_heads, s.head_dim, B, max_keys, self.dev),
        }
        self.fold_sums = fold_sums
        if fold_sums:
            # partial buffers sized for every batch the matrix cores take
            # (the split count depends on the batch)
            rows = range(16, max(B, 16) + 1)
            qb = max(gemm_q8b32_partials_bytes(b, s.qkv_dim, D) for b in rows)
            ob = max(gemm_q8b32_partials_bytes(b, D, QD) for b in rows)
            self.part_qkv = torch.empty(max(qb // 4, 4), dtype=torch.float32, device=self.dev)
            self.part_o = torch.empty(max(ob // 4, 4), dtype=torch.float32, device=self.dev)

    def step(self, X: torch.Tensor, kpool, vpool, page_table, seq_lens) -> None:
        """X: fp32 [B, D] residual rows, updated in place; kpool / vpool this
        layer's pools; seq_lens int32 [B] after the append."""
        s, B = self.s, X.shape[0]
        D, F, QD = s.dim, s.ffn_dim, s.n_heads * s.head_dim
        xn, qkv, att, h = self.xn[:B], self.qkv[:B], self.att[:B], self.h[:B]
        fold = self.fold_sums and gemm_q8b32_partials_bytes(B, s.qkv_dim, D) > 0
        ops.rmsnorm(X, self.attn_norm, s.eps, s.plus_one, y=xn, out_dtype=torch.float16)
        if fold:
            n = gemm_q8b32_partials(*self.W["wqkv"], xn, self.part_qkv)
            rope_kv_paged_sum(self.part_qkv, n, qkv, kpool, vpool, self.invf, s.n_heads, s.n_kv_heads, page_table,
                              seq_lens)
        else:
            gemm_q8b32(*self.W["wqkv"], xn, qkv, workspace=self.ws["wqkv"])
            rope_kv_paged(qkv, kpool, vpool, self.invf, s.n_heads, s.n_kv_heads, page_table, seq_lens)
        attention_paged(qkv, kpool, vpool, page_table, seq_lens, s.n_heads, self.max_keys, q_stride=s.qkv_dim,
                        out=att, workspace=self.ws["attn"])
        # the fp32 attention output and hidden rows are rounded to fp16 as the
        # products load them (the reference's attHalf / hidHalf casts)
        if fold:
            n = gemm_q8b32_partials(*self.W["wo"], att, self.part_o)
            rmsnorm_residual_sum(X, self.part_o, n, self.ffn_norm, s.eps, s.plus_one, xn)
        else:
            gemm_q8b32(*self.W["wo"], att, X, "add", workspace=self.ws["wo"])
            ops.rmsnorm(X, self.ffn_norm, s.eps, s.plus_one, y=xn, out_dtype=torch.float16)
        gemm_gate_up_q8b32(*self.W["wgate"], *self.W["wup"], xn, s.act, h, workspace=self.ws["glu"])
        gemm_q8b32(*self.W["wdown"], h, X, "add", workspace=self.ws["wdown"])


def random_layer_weights(shape: LayerShape, seed: int, std: float = 0.02) -> dict:
    """int8 block-32 weights quantised from N(0, std^2) fp16 draws (the same
    numpy quantiser as quant.quantize_q8b32), fp32 norm weights near 1."""
    rng = np.random.default_rng(seed)
    s = shape
    D, F, QD = s.dim, s.ffn_dim, s.n_heads * s.head_dim
    dims = {"wqkv": (s.qkv_dim, D), "wo": (D, QD), "wgate": (F, D), "wup": (F, D), "wdown": (D, F)}
    W = {}
    for name, (M, K) in dims.items():
        W[name] = quantize_q8b32((rng.standard_normal((M, K), dtype=np.float32) * std).astype(np.float16))
    W["attn_norm"] = (1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    W["ffn_norm"] = (1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    return W
