"""GPU parity of the prefill operators against the oracle: the fp16 batched
products (gemm_f16 / gemm_f16_add / gemm_gate_up, KL/kernels.metal:376-510) on
the matrix cores and their per-row matvec fallback, and the causal multi-query
attention of a prompt chunk (KL/kernels.metal:245-305 with T > 1).

Tolerances: fp16 products are exact in fp32 and the sums are fp32, so against
the fp64 oracle the expected error is TOL_FP32 = 1e-4 relative to max|ref|
(the contract is 1e-2)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ops as ref
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-4


def _ops():
    from gemmagemini4hackathon2026_10_2425_amd import ops

    return ops


def _close(got, want, tol=TOL_FP32):
    e = rel_err(got, want)
    assert e <= 1e-2, f"relative error {e:.3e} above the 1e-2 contract"
    assert e <= tol, f"relative error {e:.3e} above the expected {tol:.0e}"


def _wx(rng, B, M, K):
    W = (rng.standard_normal((M, K), dtype=np.float32) * 0.02).astype(np.float16)
    X = rng.standard_normal((B, K), dtype=np.float32).astype(np.float16)
    return W, X


# B rows x M x K: 16 rows (the matrix-core threshold), one and several
# 64-row activation tiles with ragged tails, weight-row tiles that leave a
# partial group of eight (the XCD-ordered grid), chunk counts 4 does not
# divide (K = 128, 256: one workgroup chunk; 384, 640: one-chunk splits),
# 12 and 6 chunks per workgroup (K = 1536, 768), and the per-row fallbacks
# (B < 16; K not a multiple of 128).
SHAPES = [(16, 640, 512), (64, 2048, 2048), (130, 640, 1024), (257, 1280, 2048), (48, 1536, 256), (20, 640, 128),
          (70, 384, 384), (33, 640, 640), (256, 4096, 1536), (256, 4096, 768), (5, 640, 512), (40, 384, 1000)]


@pytest.mark.parametrize("B,M,K", SHAPES)
@pytest.mark.parametrize("epi", ["store", "add"])
def test_gemm_f16(dev, rng, B, M, K, epi):
    ops = _ops()
    W, X = _wx(rng, B, M, K)
    base = rng.standard_normal((B, M), dtype=np.float32)
    Y = torch.from_numpy(base.copy()).to(dev)
    ops.gemm_f16(torch.from_numpy(W).to(dev), torch.from_numpy(X).to(dev), Y, epi)
    want = ref.matvec(W, X.T).T + (base.astype(np.float64) if epi == "add" else 0.0)
    _close(Y.cpu().numpy(), want)


@pytest.mark.parametrize("B,K", [(7, 2048), (64, 2048), (256, 16384), (64, 256), (40, 520)])
def test_gemm_f16_fp32_activations(dev, rng, B, K):
    """fp32 X is rounded to fp16 as the product loads it: on the matrix cores
    the result equals the product of the fp16-cast X bit for bit when both
    run the same tiling (fp16 X takes 128-row activation tiles from 256 rows,
    fp32 X keeps 64, so GM_BT = 64 lines them up); the per-row matvecs (below
    16 rows, or K % 128 != 0) sum the same fp16 values in another instruction
    order; all match the oracle on fp16(X)."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    ops = _ops()
    M = 384
    W = (rng.standard_normal((M, K), dtype=np.float32) * 0.02).astype(np.float16)
    X = rng.standard_normal((B, K), dtype=np.float32) * 3
    Wd = torch.from_numpy(W).to(dev)
    got = ops.gemm_f16(Wd, torch.from_numpy(X).to(dev)).cpu().numpy()
    cast_default = ops.gemm_f16(Wd, torch.from_numpy(X.astype(np.float16)).to(dev)).cpu().numpy()
    _lib.set_tunable("GM_BT", 64)
    try:
        cast = ops.gemm_f16(Wd, torch.from_numpy(X.astype(np.float16)).to(dev)).cpu().numpy()
    finally:
        _lib.set_tunable("GM_BT", 0)
    if B >= 16 and K % 128 == 0:
        assert np.array_equal(got, cast)
    else:
        assert np.abs(got - cast).max() <= 1e-6 * np.abs(cast).max()
    assert np.abs(cast_default - cast).max() <= 1e-6 * np.abs(cast).max()
    _close(got, ref.matvec(W, X.astype(np.float16).T).T)


@pytest.mark.parametrize("nch", [4, 8, 16, 32])
def test_gemm_f16_k_splits(dev, rng, nch):
    """Every chunk count per workgroup, so K splits into 8..1 pieces whose
    partials the reduction adds in order."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    ops = _ops()
    B, M, K = 100, 768, 4096
    W, X = _wx(rng, B, M, K)
    Wd, Xd = torch.from_numpy(W).to(dev), torch.from_numpy(X).to(dev)
    want = ref.matvec(W, X.T).T
    try:
        _lib.set_tunable("GM_NCH", nch)
        _close(ops.gemm_f16(Wd, Xd).cpu().numpy(), want)
    finally:
        _lib.set_tunable("GM_NCH", 0)


@pytest.mark.parametrize("B,F,K", [(16, 640, 512), (70, 1024, 2048), (300, 512, 1024), (32, 512, 256), (256, 4096, 1536),
                                   (8, 640, 512)])
@pytest.mark.parametrize("act", ["gelu_tanh", "silu"])
def test_gemm_gate_up_f16(dev, rng, B, F, K, act):
    ops = _ops()
    Wg, X = _wx(rng, B, F, K)
    Wu = (rng.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    H = ops.gemm_gate_up(torch.from_numpy(Wg).to(dev), torch.from_numpy(Wu).to(dev), torch.from_numpy(X).to(dev), act)
    _close(H.cpu().numpy(), ref.gate_up(Wg, Wu, X.T, act).T)


@pytest.mark.parametrize("nh,nkv,hd", [(8, 1, 256), (32, 8, 128), (4, 4, 128), (16, 8, 256), (32, 8, 64)])
@pytest.mark.parametrize("pos0,rows", [(0, 1), (0, 37), (40, 64), (100, 130)])
def test_attention_prefill(dev, rng, nh, nkv, hd, pos0, rows):
    """Query t of the chunk sees exactly keys [0, pos0 + t]: the cache past the
    chunk holds NaN/Inf, which must not leak; q rows sit inside wider qkv rows."""
    ops = _ops()
    max_ctx = 256
    kc = rng.standard_normal((nkv, max_ctx, hd), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((nkv, max_ctx, hd), dtype=np.float32).astype(np.float16)
    kc_g, vc_g = kc.copy(), vc.copy()
    kc_g[:, pos0 + rows :, :] = np.float16(np.nan)
    vc_g[:, pos0 + rows :, :] = np.float16(np.inf)
    stride = (nh + 2 * nkv) * hd
    qkv = rng.standard_normal((rows, stride), dtype=np.float32)
    out = ops.attention_prefill(torch.from_numpy(qkv).to(dev), torch.from_numpy(ops.to_tiles(kc_g, "k")).to(dev),
                                torch.from_numpy(ops.to_tiles(vc_g, "v")).to(dev), pos0, nh).cpu().numpy()
    scale = 1 / math.sqrt(hd)
    want = np.stack([ref.attention(qkv[t, : nh * hd], kc, vc, pos0 + t + 1, nh, scale) for t in range(rows)])
    _close(out, want, 1e-3)


def test_attention_prefill_rejects_bad_ranges(dev):
    from gemmagemini4hackathon2026_10_2425_amd._lib import MxdValueError

    ops = _ops()
    kc = torch.zeros((1, 64, 128), dtype=torch.float16, device=dev)
    q = torch.zeros((4, 8 * 128), dtype=torch.float32, device=dev)
    with pytest.raises(MxdValueError):
        ops.attention_prefill(q, kc, kc, 61, 8)  # positions 61..64 pass max_ctx 64
    with pytest.raises(MxdValueError):
        ops.attention_prefill(q, kc, kc, -1, 8)
