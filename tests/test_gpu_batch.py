"""GPU parity of the ragged-batch path over the paged KV cache against the
oracle: paged RoPE + append, paged split-L attention, the int8 block-32
batched products (matrix cores from 16 rows, matvec per row below) and a
whole Llama-shaped layer stepping a ragged batch, up to the full shape of 64
sequences with KV lengths uniform in [128, 8192].

Tolerances: relative 1e-4 on single-op fp32 outputs; 2e-3 on a whole layer
(three fp16 roundings of activations can land one ulp apart between the GPU's
fp32 and the oracle's fp64 arithmetic); appended cache entries within one fp16
ulp. The contract is 1e-2. From 16 rows the int8 products run on the matrix
cores with each dequantised weight rounded to fp16 (q * s, one rounding): they
are held to 1e-4 against the oracle's same rounding (oracle.batch f16_weights)
and to 1e-3 against the exact products; below 16 rows the per-row matvecs keep
the exact products (1e-4).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import batch as obatch
from oracle import ops as ref
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32


def _d(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bm():
    from gemmagemini4hackathon2026_10_2425_amd import batch

    return batch


def _f16_close(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 6e-5)) <= 2**-10


def _cache_with_rows(dev, rng, lens, nkv, hd, seed=11, stale=float("nan")):
    """A one-layer page pool whose unused slots hold `stale`, with random rows
    at positions 0..len-1 of every sequence; returns the cache and the rows."""
    B = _bm()
    table, n_pages = B.pack_ragged(lens, seed=seed)
    cache = B.PagedCache(1, nkv, hd, table, n_pages, device=dev)
    cache.k.fill_(stale)
    cache.v.fill_(stale)
    rows = []
    for b, n in enumerate(lens):
        k = rng.standard_normal((nkv, n, hd), dtype=F32).astype(F16)
        v = rng.standard_normal((nkv, n, hd), dtype=F32).astype(F16)
        cache.write(0, b, k, v)
        rows.append((k, v))
    return cache, rows


@pytest.fixture(params=["balanced", "splits"])
def schedule(request):
    """The paged attention's two schedules: items dealt evenly over the
    resident workgroups (the default up to 2048 sequences), or a fixed number
    of splits per sequence."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    _lib.set_tunable("ATT_SCHED", 1 if request.param == "balanced" else 2)
    try:
        yield request.param
    finally:
        _lib.set_tunable("ATT_SCHED", 0)


def _check_paged(dev, rng, lens, nh, nkv, hd, max_keys=None, tol=1e-4):
    B = _bm()
    cache, rows = _cache_with_rows(dev, rng, [max(n, 1) for n in lens], nkv, hd)
    q = rng.standard_normal((len(lens), nh * hd), dtype=F32)
    seq = _d(np.array(lens, np.int32), dev)
    out = B.attention_paged(_d(q, dev), cache.k[0], cache.v[0], cache.table, seq, nh,
                            max_keys=max_keys or max(max(lens), 1))
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    for b, n in enumerate(lens):
        if n == 0:
            assert (got[b] == 0).all(), b
            continue
        want = ref.attention(q[b], rows[b][0], rows[b][1], n, nh, 1.0 / math.sqrt(hd))
        assert rel_err(got[b], want) <= tol, (b, n)


@pytest.mark.parametrize("nh,nkv,hd", [(32, 8, 128), (8, 1, 256), (16, 16, 128), (32, 8, 64)])
@pytest.mark.parametrize("max_keys", [None, 32])
def test_attention_paged(dev, rng, schedule, nh, nkv, hd, max_keys):
    """Ragged lengths around page and block edges, shuffled pages, NaN in every
    unused slot; max_keys below the longest sequence only changes the split
    count, never the result."""
    _check_paged(dev, rng, [1, 15, 16, 17, 31, 32, 33, 100, 513, 2048, 5000], nh, nkv, hd, max_keys)


def test_attention_paged_empty_sequence_and_strided_q(dev, rng, schedule):
    """A sequence with no keys gets zeros; q read from qkv rows (stride > NH*hd)."""
    B = _bm()
    nh, nkv, hd = 8, 2, 128
    lens = [0, 40, 7]
    cache, rows = _cache_with_rows(dev, rng, [max(n, 1) for n in lens], nkv, hd)
    stride = (nh + 2 * nkv) * hd
    qkv = rng.standard_normal((len(lens), stride), dtype=F32)
    out = B.attention_paged(_d(qkv, dev), cache.k[0], cache.v[0], cache.table, _d(np.array(lens, np.int32), dev),
                            nh, max_keys=40, q_stride=stride).cpu().numpy()
    assert (out[0] == 0).all()
    for b in (1, 2):
        want = ref.attention(qkv[b, : nh * hd], rows[b][0], rows[b][1], lens[b], nh, 1.0 / math.sqrt(hd))
        assert rel_err(out[b], want) <= 1e-4


@pytest.mark.parametrize("per_cu", [1, 3, 64])
def test_attention_paged_balanced_pieces(dev, rng, per_cu):
    """The balanced schedule with few and with many workgroups: workgroup
    ranges that hold several whole sequences, ranges that cut one segment into
    many pieces, empty sequences between them, and a last sequence that ends
    exactly on a workgroup edge."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    lens = [0, 3, 33, 0, 0, 64, 1, 900, 31, 0, 257, 2, 4096, 17, 0]
    _lib.set_tunable("ATT_SKWG", per_cu)
    try:
        _check_paged(dev, rng, lens, 16, 4, 128)
        _check_paged(dev, rng, [0, 0, 0], 8, 2, 128)  # no keys at all: every output zero
    finally:
        _lib.set_tunable("ATT_SKWG", 0)


def test_attention_paged_many_sequences(dev, rng):
    """Past 2048 sequences the paged attention falls back to per-sequence
    splits; both sides of that edge, with short ragged lengths."""
    for n_seqs in (2048, 2049):
        lens = [int(n) for n in rng.integers(0, 70, n_seqs)]
        _check_paged(dev, rng, lens, 8, 2, 128)


def test_rope_kv_paged(dev, rng):
    B = _bm()
    nh, nkv, hd = 32, 8, 128
    lens = [1, 16, 17, 40, 300]  # keys after the append: the new token sits at len - 1
    table, n_pages = B.pack_ragged(lens, seed=5)
    cache = B.PagedCache(1, nkv, hd, table, n_pages, device=dev)
    qkv = rng.standard_normal((len(lens), (nh + 2 * nkv) * hd), dtype=F32)
    invf = ref.inv_freq(hd, 10000.0)
    qkv_d = _d(qkv, dev)
    B.rope_kv_paged(qkv_d, cache.k[0], cache.v[0], _d(invf, dev), nh, nkv, cache.table,
                    _d(np.array(lens, np.int32), dev))
    got = qkv_d.cpu().numpy()
    for b, n in enumerate(lens):
        kc = np.zeros((nkv, n, hd), F16)
        vc = np.zeros((nkv, n, hd), F16)
        q_want = ref.rope_kv(qkv[b], kc, vc, invf, nh, nkv, n - 1)
        assert rel_err(got[b, : nh * hd], q_want) <= 1e-5
        k_rows, v_rows = cache.read(0, b, n)
        _f16_close(k_rows[:, n - 1], kc[:, n - 1])
        _f16_close(v_rows[:, n - 1], vc[:, n - 1])
        assert not k_rows[:, : n - 1].any() and not v_rows[:, : n - 1].any()  # only the new position written


def _qweights(rng, M, K):
    from gemmagemini4hackathon2026_10_2425_amd.quant import quantize_q8b32

    return quantize_q8b32((rng.standard_normal((M, K), dtype=F32) * 0.02).astype(F16))


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 64, 100])
@pytest.mark.parametrize("M,K", [(1000, 4096), (96, 256), (257, 4160), (130, 640)])
def test_gemm_q8b32(dev, rng, rows, M, K):
    """Both sides of the matvec/matrix-core switch (16 rows; K % 128 for the
    matrix cores), both epilogues, the unrolled kernel (K = 4096) and the
    runtime loop (256 and 640: 2 and 5 chunks, which 4 does not divide)."""
    B = _bm()
    q, s = _qweights(rng, M, K)
    X = rng.standard_normal((rows, K), dtype=F32).astype(F16)
    mc = rows >= 16 and K % 128 == 0
    want = obatch.gemm_q8b32(q, s, X, f16_weights=mc)
    qd, sd, Xd = _d(q, dev), _d(s, dev), _d(X, dev)
    got = B.gemm_q8b32(qd, sd, Xd).cpu().numpy()
    assert rel_err(got, want) <= 1e-4
    assert rel_err(got, obatch.gemm_q8b32(q, s, X)) <= 1e-3
    Y0 = rng.standard_normal((rows, M), dtype=F32)
    Yd = _d(Y0, dev)
    B.gemm_q8b32(qd, sd, Xd, Yd, "add")
    assert rel_err(Yd.cpu().numpy(), Y0 + want) <= 1e-4


@pytest.mark.parametrize("rows,K", [(5, 4096), (64, 4096), (64, 14336), (37, 640)])
def test_gemm_q8b32_fp32_activations(dev, rng, rows, K):
    """fp32 X is rounded to fp16 as the product loads it: on the matrix cores
    (the unrolled kernel, the runtime loop) the result equals the product of the
    fp16-cast X bit for bit; the per-row matvecs below 16 rows sum the same
    fp16 values in another instruction order (fp32 FMAs, not packed dot
    products); both match the oracle on fp16(X)."""
    B = _bm()
    M = 512
    q, s = _qweights(rng, M, K)
    X = rng.standard_normal((rows, K), dtype=F32) * 3
    qd, sd = _d(q, dev), _d(s, dev)
    got = B.gemm_q8b32(qd, sd, _d(X, dev)).cpu().numpy()
    cast = B.gemm_q8b32(qd, sd, _d(X.astype(F16), dev)).cpu().numpy()
    if rows >= 16:
        assert np.array_equal(got, cast)
    else:
        assert rel_err(got, cast) <= 1e-6
    assert rel_err(got, obatch.gemm_q8b32(q, s, X.astype(F16), f16_weights=rows >= 16)) <= 1e-4


@pytest.mark.parametrize("nch,splits", [(4, 0), (8, 0), (16, 0), (32, 0), (1, 1), (1, 3), (1, 32)])
def test_gemm_q8b32_k_splits(dev, rng, nch, splits):
    """Every chunk count of the unrolled kernel (8, 4, 2 and 1 K splits at K =
    4096) and the runtime loop (GM_NCH = 1) at 1, 3 and 32 splits; partials
    are added in split order by the second kernel."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    B = _bm()
    M, K, rows = 300, 4096, 40
    q, s = _qweights(rng, M, K)
    X = rng.standard_normal((rows, K), dtype=F32).astype(F16)
    want = obatch.gemm_q8b32(q, s, X, f16_weights=True)
    try:
        _lib.set_tunable("GM_NCH", nch)
        _lib.set_tunable("GM_SPLITS", splits)
        Y0 = rng.standard_normal((rows, M), dtype=F32)
        Yd = _d(Y0, dev)
        B.gemm_q8b32(_d(q, dev), _d(s, dev), _d(X, dev), Yd, "add")
        assert rel_err(Yd.cpu().numpy(), Y0 + want) <= 1e-4
    finally:
        _lib.set_tunable("GM_NCH", 0)
        _lib.set_tunable("GM_SPLITS", 0)


@pytest.mark.parametrize("rows", [8, 16, 64])
@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_gemm_gate_up_q8b32(dev, rng, rows, act):
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    B = _bm()
    F, K = 1000, 1024
    qg, sg = _qweights(rng, F, K)
    qu, su = _qweights(rng, F, K)
    X = rng.standard_normal((rows, K), dtype=F32).astype(F16)
    want = obatch.gate_up_rows(qg, sg, qu, su, X, act, f16_weights=rows >= 16)
    args = [_d(a, dev) for a in (qg, sg, qu, su, X)]
    # as chosen (4 chunks, 2 splits), one split of 8 unrolled chunks, and the
    # runtime loop with and without partials
    for nch, splits in ((0, 0), (8, 0), (1, 1), (1, 4)):
        try:
            _lib.set_tunable("GM_NCH", nch)
            _lib.set_tunable("GM_SPLITS", splits)
            assert rel_err(B.gemm_gate_up_q8b32(*args, act).cpu().numpy(), want) <= 1e-4
        finally:
            _lib.set_tunable("GM_NCH", 0)
            _lib.set_tunable("GM_SPLITS", 0)


@pytest.mark.parametrize("rows,M,K,xdt", [(16, 6144, 4096, F16), (64, 4096, 4096, F32), (64, 4096, 14336, F32),
                                           (37, 300, 1024, F16), (100, 257, 640, F32)])
def test_gemm_q8b32_partials_sum_to_the_product(dev, rng, rows, M, K, xdt):
    """The unsummed K-split partials, added in split order from zero, are
    bit-identical to the summing product (store and add epilogues)."""
    B = _bm()
    q, s = _qweights(rng, M, K)
    X = rng.standard_normal((rows, K), dtype=F32).astype(xdt)
    qd, sd, Xd = _d(q, dev), _d(s, dev), _d(X, dev)
    part = torch.empty(B.gemm_q8b32_partials_bytes(rows, M, K) // 4, dtype=torch.float32, device=dev)
    n = B.gemm_q8b32_partials(qd, sd, Xd, part)
    assert n >= 1 and part.numel() == n * rows * M
    P = part.cpu().numpy().reshape(n, rows, M)
    acc = np.zeros((rows, M), F32)
    for sp in range(n):
        acc = acc + P[sp]
    assert np.array_equal(acc, B.gemm_q8b32(qd, sd, Xd).cpu().numpy())
    base = rng.standard_normal((rows, M), dtype=F32)
    Y = _d(base, dev)
    B.gemm_q8b32(qd, sd, Xd, Y, "add")
    assert np.array_equal(base + acc, Y.cpu().numpy())


def test_gemm_q8b32_partials_rejects_small_batches(dev, rng):
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    B = _bm()
    q, s = _qweights(rng, 64, 256)
    X = _d(rng.standard_normal((15, 256), dtype=F32).astype(F16), dev)
    assert B.gemm_q8b32_partials_bytes(15, 64, 256) == 0
    with pytest.raises(_lib.MxdValueError):
        B.gemm_q8b32_partials(_d(q, dev), _d(s, dev), X, torch.empty(64 * 15, dtype=torch.float32, device=dev))


def test_ops_that_add_partials_match_the_summing_path(dev, rng):
    """rope_kv_paged_sum and rmsnorm_residual_sum over a product's partials give
    bit for bit what the summing product followed by rope_kv_paged / rmsnorm
    gives (q, the appended k and v, the residual and the normed rows)."""
    from gemmagemini4hackathon2026_10_2425_amd import ops

    B = _bm()
    nh, nkv, hd, D = 8, 2, 128, 1024
    lens = [int(n) for n in np.random.default_rng(7).integers(1, 200, 18)] + [1, 16]  # 20 rows: matrix cores
    rows, QKV = len(lens), (nh + 2 * nkv) * hd
    invf = _d(ref.inv_freq(hd, 10000.0), dev)
    seq = _d(np.array(lens, np.int32), dev)
    q, s = _qweights(rng, QKV, D)
    qd, sd = _d(q, dev), _d(s, dev)
    xn = _d(rng.standard_normal((rows, D), dtype=F32).astype(F16), dev)
    part = torch.empty(B.gemm_q8b32_partials_bytes(rows, QKV, D) // 4, dtype=torch.float32, device=dev)
    n = B.gemm_q8b32_partials(qd, sd, xn, part)
    caches = []
    for _ in range(2):
        table, n_pages = B.pack_ragged(lens, seed=9)
        caches.append(B.PagedCache(1, nkv, hd, table, n_pages, device=dev))
    qkv_a = torch.zeros((rows, QKV), dtype=torch.float32, device=dev)
    B.rope_kv_paged_sum(part, n, qkv_a, caches[0].k[0], caches[0].v[0], invf, nh, nkv, caches[0].table, seq)
    qkv_b = B.gemm_q8b32(qd, sd, xn)
    B.rope_kv_paged(qkv_b, caches[1].k[0], caches[1].v[0], invf, nh, nkv, caches[1].table, seq)
    torch.cuda.synchronize()
    assert torch.equal(qkv_a[:, : nh * hd], qkv_b[:, : nh * hd])
    assert torch.equal(caches[0].k, caches[1].k) and torch.equal(caches[0].v, caches[1].v)

    qo, so = _qweights(rng, D, nh * hd)
    att = _d(rng.standard_normal((rows, nh * hd), dtype=F32), dev)
    w = _d((1.0 + 0.02 * rng.standard_normal(D)).astype(F32), dev)
    X = rng.standard_normal((rows, D), dtype=F32)
    part_o = torch.empty(B.gemm_q8b32_partials_bytes(rows, D, nh * hd) // 4, dtype=torch.float32, device=dev)
    no = B.gemm_q8b32_partials(_d(qo, dev), _d(so, dev), att, part_o)
    for plus_one, ydt in ((False, torch.float16), (True, torch.float32)):
        Xa, Xb = _d(X, dev), _d(X, dev)
        ya = torch.empty((rows, D), dtype=ydt, device=dev)
        B.rmsnorm_residual_sum(Xa, part_o, no, w, 1e-5, plus_one, ya)
        B.gemm_q8b32(_d(qo, dev), _d(so, dev), att, Xb, "add")
        yb = ops.rmsnorm(Xb, w, 1e-5, plus_one, out_dtype=ydt)
        assert torch.equal(Xa, Xb) and torch.equal(ya, yb)


def test_ragged_layer_fold_sums_is_bit_exact(dev):
    """The layer step with the qkv and o sums folded into the next ops equals
    the step with summing products, bit for bit (residual rows and pools)."""
    from gemmagemini4hackathon2026_10_2425_amd import ops

    B = _bm()
    shape = B.LayerShape(dim=512, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=1024)
    lens = [int(n) for n in np.random.default_rng(8).integers(1, 300, 24)]
    W = B.random_layer_weights(shape, 8)
    X = np.random.default_rng(8).standard_normal((len(lens), shape.dim), dtype=F32)
    out = []
    for fold in (True, False):
        table, n_pages = B.pack_ragged(lens, seed=8)
        cache = B.PagedCache(1, shape.n_kv_heads, shape.head_dim, table, n_pages, device=dev)
        for pool, tid in ((cache.k, 1), (cache.v, 2)):
            pool.copy_(ops.fill_normal(tuple(pool.shape), torch.float16, 8, tid, 1.0, dev))
        layer = B.RaggedLayerQ8(shape, W, max_batch=len(lens), max_keys=max(lens), device=dev, fold_sums=fold)
        Xd = _d(X, dev)
        layer.step(Xd, cache.k[0], cache.v[0], cache.table, _d(np.array(lens, np.int32), dev))
        torch.cuda.synchronize()
        out.append((Xd.cpu(), cache.k.cpu(), cache.v.cpu()))
    for a, b in zip(*out):
        assert torch.equal(a, b)


def _layer_parity(dev, shape, lens, seed):
    """Step a ragged batch through RaggedLayerQ8 and through the oracle; compare
    the new residual rows and every sequence's appended K/V."""
    from gemmagemini4hackathon2026_10_2425_amd import ops

    B = _bm()
    ocfg = obatch.LayerConfig(shape.dim, shape.n_heads, shape.n_kv_heads, shape.head_dim, shape.ffn_dim,
                              shape.eps, shape.rope_theta, shape.act, shape.plus_one)
    W = B.random_layer_weights(shape, seed)
    table, n_pages = B.pack_ragged(lens, seed=seed)
    cache = B.PagedCache(1, shape.n_kv_heads, shape.head_dim, table, n_pages, device=dev)
    for pool, tid in ((cache.k, 1), (cache.v, 2)):  # every slot random, as a long-lived pool would hold
        pool.copy_(ops.fill_normal(tuple(pool.shape), torch.float16, seed, tid, 1.0, dev))
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((len(lens), shape.dim), dtype=F32)
    kc, vc = zip(*[cache.read(0, b, n) for b, n in enumerate(lens)])
    kc, vc = [k.copy() for k in kc], [v.copy() for v in vc]
    want = obatch.layer_step(ocfg, W, X, kc, vc, np.array(lens), f16_weights=len(lens) >= 16)

    layer = B.RaggedLayerQ8(shape, W, max_batch=len(lens), max_keys=max(lens), device=dev)
    Xd = _d(X, dev)
    layer.step(Xd, cache.k[0], cache.v[0], cache.table, _d(np.array(lens, np.int32), dev))
    got = Xd.cpu().numpy()
    assert rel_err(got, want) <= 2e-3
    for b, n in enumerate(lens):
        k, v = cache.read(0, b, n)
        # the appended k/v derive from the fp16 normed activations, so they
        # carry the same few-ulp spread as the outputs
        assert rel_err(k[:, n - 1], kc[b][:, n - 1]) <= 2e-3
        assert rel_err(v[:, n - 1], vc[b][:, n - 1]) <= 2e-3
        assert np.array_equal(k[:, : n - 1], kc[b][:, : n - 1])  # older positions untouched


def test_ragged_layer_small(dev):
    B = _bm()
    shape = B.LayerShape(dim=512, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=1024)
    lens = list(np.random.default_rng(3).integers(1, 300, 20)) + [1, 16, 17, 33]
    _layer_parity(dev, shape, [int(n) for n in lens], seed=3)


def test_ragged_layer_below_matrix_core_threshold(dev):
    """Fewer than 16 sequences: the same layer through the per-row matvecs."""
    B = _bm()
    shape = B.LayerShape(dim=512, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=1024)
    _layer_parity(dev, shape, [5, 100, 37], seed=4)


def test_ragged_layer_llama8b_64_sequences(dev):
    """The full batched shape: one Llama-3-8B layer (hidden 4096, 32 Q / 8 KV
    heads, head_dim 128, SwiGLU 14336, int8 block-32), 64 sequences with KV
    lengths uniform in [128, 8192] in a shuffled 16-key page pool."""
    B = _bm()
    lens = np.random.default_rng(20261201).integers(128, 8193, 64) + 1  # + this step's token
    _layer_parity(dev, B.LLAMA3_8B_LAYER, [int(n) for n in lens], seed=5)
