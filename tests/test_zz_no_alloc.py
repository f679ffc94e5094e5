"""mxd_attention_noalloc (the allocation-free attention entry point) against
mxd_attention, both called through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller input, and shapes whose partials
exceed the scratch array rejected on the host."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import ops as ref
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _case(rng, nh, nkv, hd, L, max_ctx, dev):
    from gemmagemini4hackathon2026_10_2425_amd import ops

    q = rng.standard_normal(nh * hd, dtype=np.float32)
    kc = np.zeros((nkv, max_ctx, hd), np.float16)
    vc = np.zeros((nkv, max_ctx, hd), np.float16)
    kc[:, :L] = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
    vc[:, :L] = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
    tens = [torch.from_numpy(a).to(dev) for a in (q, ops.to_tiles(kc, "k"), ops.to_tiles(vc, "v"))]
    return (q, kc, vc), tens


def _both(L_, nh, nkv, hd, max_ctx, n_keys, tens, dev):
    """(mxd_attention with a workspace, mxd_attention_noalloc) outputs."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    qd, kd, vd = tens
    scale = 1.0 / math.sqrt(hd)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    ws_bytes = _lib.query("mxd_attention_workspace_size", nh, nkv, hd, max_ctx)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    a = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device=dev)
    b = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device=dev)
    _lib.call("mxd_attention", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), a.data_ptr(), nh, nkv, hd, max_ctx, n_keys,
              None, scale, ws.data_ptr(), ws.numel(), stream)
    _lib.call("mxd_attention_noalloc", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), b.data_ptr(), nh, nkv, hd,
              max_ctx, n_keys, None, scale, stream)
    torch.cuda.synchronize(dev)
    return a.cpu().numpy(), b.cpu().numpy()


def test_attention_noalloc_matches_attention(dev):
    rng = np.random.default_rng(7)
    nh, nkv, hd = 32, 8, 128
    # a long context (96 splits of partials in the scratch array), then a
    # shorter one that leaves part of the first call's partials in place
    for L, max_ctx in ((32768, 32768), (3000, 4096), (300, 512)):
        host, tens = _case(rng, nh, nkv, hd, L, max_ctx, dev)
        a, b = _both(L, nh, nkv, hd, max_ctx, L, tens, dev)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), L
        q, kc, vc = host
        assert rel_err(b, ref.attention(q, kc, vc, L, nh, 1 / math.sqrt(hd))) <= 1e-3, L


def test_attention_noalloc_gemma_shape_twice(dev):
    rng = np.random.default_rng(8)
    nh, nkv, hd = 8, 1, 256
    for L in (8192, 1000):
        host, tens = _case(rng, nh, nkv, hd, L, 8192, dev)
        a, b = _both(L, nh, nkv, hd, 8192, L, tens, dev)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), L


def test_attention_noalloc_rejects_shapes_beyond_the_scratch(dev):
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    assert _lib.query("mxd_attention_noalloc_max_scratch") == 8 << 20
    P = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    _lib.set_tunable("ATT_WGCU", 16)
    try:
        with pytest.raises(_lib.MxdValueError) as ei:
            _lib.call("mxd_attention_noalloc", P, P, P, P, 64, 8, 256, 32768, 32768, None, 0.0625, None)
        assert ei.value.code == _lib.MXD_ERR_UNSUPPORTED and "scratch" in _lib.last_error()
    finally:
        _lib.set_tunable("ATT_WGCU", 0)
