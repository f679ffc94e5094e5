"""GPU parity of the fused decode-step operators against the oracle's unfused
composition: rmsnorm + matvec, rmsnorm + gate_up, rmsnorm + qkv + RoPE + append.

Tolerances as in test_gpu_ops: relative 1e-4 on fp32 outputs (contract 1e-2);
fp16 cache entries within one fp16 ulp (the GPU rounds its fp32 result, the
oracle its fp64 result).
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import ops as ref
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _lib():
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    return _lib


def _d(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _f16_close(got, want):
    got, want = got.astype(np.float64), want.astype(np.float64)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 6e-5)) <= 2**-10


@pytest.mark.parametrize("plus_one", [True, False])
@pytest.mark.parametrize("M,K", [(2048, 2048), (256000, 2048), (70001, 2048), (65536, 1024), (37, 4096)])
def test_matvec_rmsnorm(dev, rng, M, K, plus_one):
    """Tiled rows (small M) and, from 65536 rows of up to 4 KiB, the grid
    sweep: rows left over past the last full round of workgroups (70001) and
    rows shorter than the workgroup's waves (K = 1024: two chunks, four waves)."""
    L = _lib()
    W = (rng.standard_normal((M, K), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(K, dtype=np.float32) * 4
    w = rng.standard_normal(K, dtype=np.float32) * 0.02
    y = torch.empty(M, dtype=torch.float32, device=dev)
    Wd, xd, wd = _d(W, dev), _d(x, dev), _d(w, dev)  # keep the device copies alive across the call
    L.call("mxd_matvec_f16_rmsnorm", Wd.data_ptr(), xd.data_ptr(), wd.data_ptr(), 1e-6,
           int(plus_one), y.data_ptr(), M, K, L.MXD_EPI_STORE, None, _stream())
    xn = ref.rmsnorm(x, w, 1e-6, plus_one).astype(np.float32)
    e = rel_err(y.cpu().numpy(), ref.matvec(W, xn))
    assert e <= 1e-4


@pytest.mark.parametrize("act", ["gelu_tanh", "silu"])
def test_gate_up_rmsnorm(dev, rng, act):
    L = _lib()
    F, K = 16384, 2048
    Wg = (rng.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    Wu = (rng.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(K, dtype=np.float32) * 3
    w = rng.standard_normal(K, dtype=np.float32) * 0.02
    h = torch.empty(F, dtype=torch.float32, device=dev)
    Wgd, Wud, xd, wd = _d(Wg, dev), _d(Wu, dev), _d(x, dev), _d(w, dev)
    L.call("mxd_gate_up_rmsnorm", Wgd.data_ptr(), Wud.data_ptr(), xd.data_ptr(), wd.data_ptr(), 1e-6, 1,
           h.data_ptr(), F, K, L.MXD_ACT_SILU if act == "silu" else L.MXD_ACT_GELU_TANH, _stream())
    xn = ref.rmsnorm(x, w, 1e-6, True).astype(np.float32)
    assert rel_err(h.cpu().numpy(), ref.gate_up(Wg, Wu, xn, act)) <= 1e-4


@pytest.mark.parametrize("nh,nkv,hd,D", [(8, 1, 256, 2048), (32, 8, 128, 4096), (4, 2, 128, 256), (32, 8, 64, 2048)])
@pytest.mark.parametrize("pos", [0, 45, 383])
@pytest.mark.parametrize("device_pos", [False, True])
def test_qkv_rope_kv(dev, rng, nh, nkv, hd, D, pos, device_pos):
    from gemmagemini4hackathon2026_10_2425_amd import ops

    L = _lib()
    max_ctx = 384
    M = (nh + 2 * nkv) * hd
    W = (rng.standard_normal((M, D), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(D, dtype=np.float32) * 2
    w = rng.standard_normal(D, dtype=np.float32) * 0.02
    invf = ref.inv_freq(hd, 10000.0)
    # oracle: unfused norm -> matvec (rounded to fp32 like the GPU's qkv buffer) -> rope + append
    qkv = ref.matvec(W, ref.rmsnorm(x, w, 1e-6, True).astype(np.float32)).astype(np.float32)
    kc = np.zeros((nkv, max_ctx, hd), np.float16)
    vc = np.zeros((nkv, max_ctx, hd), np.float16)
    q_want = ref.rope_kv(qkv, kc, vc, invf, nh, nkv, pos)
    q = torch.zeros(nh * hd, dtype=torch.float32, device=dev)
    kd = torch.zeros((nkv, max_ctx, hd), dtype=torch.float16, device=dev)
    vd = torch.zeros((nkv, max_ctx, hd), dtype=torch.float16, device=dev)
    pos_t = torch.tensor([pos], dtype=torch.int32, device=dev)
    Wd, xd, wd, fd = _d(W, dev), _d(x, dev), _d(w, dev), _d(invf, dev)
    L.call("mxd_qkv_rope_kv", Wd.data_ptr(), xd.data_ptr(), wd.data_ptr(), 1e-6, 1, q.data_ptr(), kd.data_ptr(),
           vd.data_ptr(), fd.data_ptr(), nh, nkv, hd, D, max_ctx, -1 if device_pos else pos,
           pos_t.data_ptr() if device_pos else None, _stream())
    assert rel_err(q.cpu().numpy(), q_want) <= 1e-4
    k_rows = ops.from_tiles(kd.cpu().numpy(), "k")
    v_rows = ops.from_tiles(vd.cpu().numpy(), "v")
    _f16_close(k_rows[:, pos], kc[:, pos])
    _f16_close(v_rows[:, pos], vc[:, pos])
    assert np.count_nonzero(k_rows) == np.count_nonzero(k_rows[:, pos])  # only position pos written
    assert np.count_nonzero(v_rows) == np.count_nonzero(v_rows[:, pos])


@pytest.mark.parametrize("algo", [0, 1, 2])
def test_every_matvec_variant(dev, rng, algo):
    """The three matvec work layouts (row tiles, row streaming, grid sweep) give
    the oracle's answer for int8 weights, the two-matrix GLU, the fused norm
    and the residual-add epilogue, including ragged M and K tails."""
    from gemmagemini4hackathon2026_10_2425_amd import ops
    from gemmagemini4hackathon2026_10_2425_amd.quant import quantize_q8b32

    L = _lib()
    M, K = 1037, 4096 + 1024 + 64
    W = (rng.standard_normal((M, K), dtype=np.float32) * 0.02).astype(np.float16)
    Wu = (rng.standard_normal((M, K), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(K, dtype=np.float32)
    nw_ = rng.standard_normal(K, dtype=np.float32) * 0.02
    q, s = quantize_q8b32(W)
    x16 = x.astype(np.float16)
    Wd, Wud, xd, x16d, nwd = _d(W, dev), _d(Wu, dev), _d(x, dev), _d(x16, dev), _d(nw_, dev)
    qd, sd = _d(q, dev), _d(s, dev)
    try:
        L.set_tunable("MV_ALGO", algo)
        y = ops.matvec_q8b32(qd, sd, x16d)
        assert rel_err(y.cpu().numpy(), ref.matvec_q8b32(q, s, x16)) <= 1e-4
        h = ops.matvec_gate_up(Wd, Wud, xd, "silu")
        assert rel_err(h.cpu().numpy(), ref.gate_up(W, Wu, x, "silu")) <= 1e-4
        base = rng.standard_normal(M, dtype=np.float32)
        yd = _d(base, dev)
        ops.matvec_f16_add(Wd, xd, yd)
        assert rel_err(yd.cpu().numpy(), base + ref.matvec(W, x)) <= 1e-4
        yn = torch.empty(M, dtype=torch.float32, device=dev)
        L.call("mxd_matvec_f16_rmsnorm", Wd.data_ptr(), xd.data_ptr(), nwd.data_ptr(), 1e-6, 1, yn.data_ptr(), M, K,
               L.MXD_EPI_STORE, None, _stream())
        xn = ref.rmsnorm(x, nw_, 1e-6, True).astype(np.float32)
        assert rel_err(yn.cpu().numpy(), ref.matvec(W, xn)) <= 1e-4
    finally:
        L.set_tunable("MV_ALGO", 0)


@pytest.mark.parametrize("nh,nkv,hd,M", [(8, 1, 256, 2048), (32, 8, 128, 4096), (4, 2, 128, 300), (32, 8, 64, 2048)])
@pytest.mark.parametrize("L,n_splits", [(1, 3), (45, 3), (384, 3), (129, 8), (1000, 8), (700, 2)])
@pytest.mark.parametrize("device_pos", [False, True])
def test_attention_split_merged_by_matvec(dev, rng, nh, nkv, hd, M, L, n_splits, device_pos):
    """Attention left as unmerged split partials, merged by the o projection
    as it loads its input, equals the oracle's attention then matvec + residual;
    cache rows past the key count hold NaN/inf and must not leak."""
    from gemmagemini4hackathon2026_10_2425_amd import ops

    max_ctx = 1024
    q = rng.standard_normal(nh * hd, dtype=np.float32)
    kc = np.full((nkv, max_ctx, hd), np.nan, np.float16)
    vc = np.full((nkv, max_ctx, hd), np.inf, np.float16)
    kc[:, :L] = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
    vc[:, :L] = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
    W = (rng.standard_normal((M, nh * hd), dtype=np.float32) * 0.02).astype(np.float16)
    base = rng.standard_normal(M, dtype=np.float32)
    qd, kd, vd = _d(q, dev), _d(ops.to_tiles(kc, "k"), dev), _d(ops.to_tiles(vc, "v"), dev)
    Wd, yd = _d(W, dev), _d(base, dev)
    pos = torch.tensor([L - 1], dtype=torch.int32, device=dev) if device_pos else None
    n_keys = 0 if device_pos else L
    part = ops.attention_split(qd, kd, vd, n_keys, nh, n_splits, pos_dev=pos)
    ops.matvec_f16_attn_merge(Wd, part, n_splits, nh, hd, max_ctx, n_keys, y=yd, epilogue="add", pos_dev=pos)
    att = ref.attention(q, kc[:, :L], vc[:, :L], L, nh, 1 / math.sqrt(hd)).astype(np.float32)
    want = base + ref.matvec(W, att)
    assert rel_err(yd.cpu().numpy(), want) <= 1e-3


def test_attention_split_rejects_bad_args(dev):
    from gemmagemini4hackathon2026_10_2425_amd import _lib as L
    from gemmagemini4hackathon2026_10_2425_amd import ops

    q = torch.zeros(8 * 256, dtype=torch.float32, device=dev)
    kc = torch.zeros((1, 64, 256), dtype=torch.float16, device=dev)
    with pytest.raises(L.MxdValueError):
        ops.attention_split(q, kc, kc, 10, 8, 600)  # more splits than supported
    part = ops.attention_split(q, kc, kc, 10, 8, 2)
    W = torch.zeros((16, 8 * 256), dtype=torch.float16, device=dev)
    with pytest.raises(L.MxdValueError):
        ops.matvec_f16_attn_merge(W, part, 9, 8, 256, 64, 10)  # the merge takes at most 8 splits
