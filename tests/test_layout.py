"""The tiled KV-cache layout (include/mxdecode.h) on the CPU: offsets are a
permutation inside each 32-position tile, and the helpers invert each other."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gemmagemini4hackathon2026_10_2425_amd import ops


@pytest.mark.parametrize("hd", [128, 256])
@pytest.mark.parametrize("which", ["k", "v"])
def test_offsets_are_a_tilewise_permutation(hd, which):
    ctx = 96
    off = ops.tile_offsets(ctx, hd, which)
    assert np.array_equal(np.sort(off.reshape(-1)), np.arange(ctx * hd))
    for p in range(ctx):
        lo = (p // 32) * 32 * hd
        assert off[p].min() >= lo and off[p].max() < lo + 32 * hd


@pytest.mark.parametrize("which", ["k", "v"])
def test_operand_chunks_are_contiguous(which):
    """Each 1 KiB chunk of a tile is one MFMA operand load: lane l's 8 halfs."""
    hd = 128
    off = ops.tile_offsets(32, hd, which)
    if which == "v":
        # chunk d, lane (col=dim&15, g=key>>3): keys 8g..8g+7 of dim 16d+col
        for d in range(hd // 16):
            for lane in range(64):
                col, g = lane & 15, lane >> 4
                got = off[8 * g : 8 * g + 8, 16 * d + col]
                assert np.array_equal(got, d * 512 + lane * 8 + np.arange(8))
    else:
        for t in range(2):
            for c in range(hd // 32):
                for lane in range(64):
                    col, g = lane & 15, lane >> 4
                    key = 8 * (col >> 2) + 4 * t + (col & 3)
                    got = off[key, 32 * c + 8 * g : 32 * c + 8 * g + 8]
                    assert np.array_equal(got, (t * (hd // 32) + c) * 512 + lane * 8 + np.arange(8))


def test_to_from_tiles_roundtrip():
    rng = np.random.default_rng(0)
    rows = rng.standard_normal((3, 64, 128)).astype(np.float16)
    for which in ("k", "v"):
        t = ops.to_tiles(rows, which)
        assert np.array_equal(ops.from_tiles(t, which), rows)
        tt = ops.to_tiles(torch.from_numpy(rows), which)
        assert np.array_equal(tt.numpy(), t)
        assert np.array_equal(ops.from_tiles(tt, which).numpy(), rows)
