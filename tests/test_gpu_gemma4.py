"""Gemma-4 on the GPU against the oracle (oracle/gemma4.py, itself pinned to
transformers' Gemma4ForCausalLM): the new operators one by one (sandwich-norm
residual add, per-layer-embedding combine, per-head q/k/v norm + partial RoPE +
append, sliding-window attention and head_dim 512), then the engine on the tiny
Gemma-4 config (every feature of the reference's E2B engine at small size):
synthetic weights bit for bit, softcapped logits at every position, greedy
tokens equal to transformers' (tests/golden/hf_gemma4_tiny.npz), and the
graph-replayed decode equal to eager steps.

Tolerances: operators max|got - ref| / max|ref| <= 1e-4 (fp32 math; attention
1e-3 through its fp16 matrix-core split); the contract is 1e-2. Engine logits
<= 2e-3: the GPU and the oracle store the same fp16 K/V, but fp32 rounding
differences of ~1e-7 flip single fp16 roundings, and the model passes such
flips on to the logits the way storing K/V in fp16 at all does, which moves
the fixture model's logits by at most 6.3e-4 (oracle with fp16 against fp64
K/V over the fixture's 31 positions). The fixture's q/k norm weights are
scaled by 0.25 for that conditioning (with weight 1, unit-RMS q and k at
attention scale 1 give near one-hot softmaxes and a 1.1e-2 sensitivity).
Token ids are exact: the fixture's greedy margins exceed 2% of the largest
logit. Cache bits are exact.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gemma4 as g4
from oracle import ops as ref
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "hf_gemma4_tiny.npz"
TOL_CONTRACT = 1e-2


def _ops():
    from gemmagemini4hackathon2026_10_2425_amd import ops

    return ops


def _close(got, want, tol):
    e = rel_err(got, want)
    assert e <= TOL_CONTRACT, f"relative error {e:.3e} above the 1e-2 contract"
    assert e <= tol, f"relative error {e:.3e} above the expected {tol:.0e}"


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ---------------------------------------------------------------- operators


@pytest.mark.parametrize("rows,D", [(1, 256), (3, 1536), (2, 100)])
@pytest.mark.parametrize("post", [1.0, 0.7])
def test_rmsnorm_add(dev, rng, rows, D, post):
    src = rng.standard_normal((rows, D), dtype=np.float32) * 3
    x = rng.standard_normal((rows, D), dtype=np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    got = _ops().rmsnorm_add(_t(src, dev), _t(w, dev), _t(x, dev), 1e-6, post).cpu().numpy()
    want = (x.astype(np.float64) + g4.rmsnorm_w(src, w, 1e-6)) * post
    _close(got, want, 1e-6)


@pytest.mark.parametrize("rows,L,P,D", [(1, 6, 32, 256), (2, 35, 256, 1536)])
def test_ple_combine(dev, rng, rows, L, P, D):
    proj = rng.standard_normal((rows, L * P), dtype=np.float32) * 5
    ple = rng.standard_normal((rows, L * P), dtype=np.float32)
    w = (1 + 0.1 * rng.standard_normal(P)).astype(np.float32)
    got = _ops().ple_combine(_t(proj, dev), _t(ple, dev), _t(w, dev), L, D, 1e-6).cpu().numpy()
    p = proj.reshape(rows, L, P).astype(np.float64) * np.float32(D ** -0.5)
    want = (g4.rmsnorm_w(p, w, 1e-6) + ple.reshape(rows, L, P)) * 2 ** -0.5
    _close(got.reshape(rows, L, P), want, 1e-6)


@pytest.mark.parametrize("M,K", [(2560, 1536), (256, 1536), (65536, 1536), (1024, 256), (6144, 1536)])
@pytest.mark.parametrize("norm", [True, False])
def test_matvec_residual(dev, rng, M, K, norm):
    """The sandwich norm's residual add folded into the next product: x_out =
    (x + rmsnorm(src) * w) * post, y = W . rmsnorm(x_out) * nw (or W . x_out
    with the gelu * aux epilogue); every tiling the shape selects, the LM-head
    sweep included."""
    ops = _ops()
    x = rng.standard_normal(K, dtype=np.float32)
    src = rng.standard_normal(K, dtype=np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((M, K), dtype=np.float32) * 0.02).astype(np.float16)
    aux = rng.standard_normal(M, dtype=np.float32)
    xw = (x.astype(np.float64) + g4.rmsnorm_w(src, w, 1e-6)) * 0.7
    xo = torch.empty(K, dtype=torch.float32, device=dev)
    if norm:
        y = ops.matvec_f16_residual(_t(W, dev), _t(x, dev), _t(src, dev), _t(w, dev), xo, 1e-6, 0.7, _t(nw, dev))
        want = ref.matvec(W, g4.rmsnorm_w(xw, nw, 1e-6))
    else:
        y = ops.matvec_f16_residual(_t(W, dev), _t(x, dev), _t(src, dev), _t(w, dev), xo, 1e-6, 0.7,
                                    epilogue="gelu_mul", aux=_t(aux, dev))
        want = ref.gelu_tanh(ref.matvec(W, xw)) * aux
    _close(xo.cpu().numpy(), xw, 1e-6)
    _close(y.cpu().numpy(), want, 1e-5)


@pytest.mark.parametrize("F,K", [(6144, 1536), (512, 256)])
def test_gate_up_residual(dev, rng, F, K):
    ops = _ops()
    x = rng.standard_normal(K, dtype=np.float32)
    src = rng.standard_normal(K, dtype=np.float32)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wg = (rng.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    Wu = (rng.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    xo = torch.empty(K, dtype=torch.float32, device=dev)
    h = ops.gate_up_residual(_t(Wg, dev), _t(Wu, dev), _t(x, dev), _t(src, dev), _t(w, dev), xo, _t(nw, dev), 1e-6)
    xw = x.astype(np.float64) + g4.rmsnorm_w(src, w, 1e-6)
    _close(xo.cpu().numpy(), xw, 1e-6)
    _close(h.cpu().numpy(), ref.gate_up(Wg, Wu, g4.rmsnorm_w(xw, nw, 1e-6), "gelu_tanh"), 1e-5)


def _tile_rows(tiles, pos, which):
    """Cache rows [n_kv, hd] at position pos of the tiled layout."""
    ops = _ops()
    n_kv, ctx, hd = tiles.shape
    off = ops.tile_offsets(ctx, hd, which)[pos]
    return tiles.reshape(n_kv, -1)[:, off]


@pytest.mark.parametrize("nh,nkv,hd,pairs", [(8, 1, 256, 128), (8, 1, 512, 64), (4, 1, 64, 32), (4, 2, 128, 16),
                                             (8, 0, 512, 64), (4, 0, 64, 32)])
@pytest.mark.parametrize("pos", [0, 17, 1023])
def test_qk_norm_rope_kv(dev, rng, nh, nkv, hd, pairs, pos):
    ops = _ops()
    max_ctx = 1024
    qkv = rng.standard_normal((nh + 2 * nkv) * hd, dtype=np.float32) * 2
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    i = np.arange(hd // 2, dtype=np.float64)
    invf = np.where(i < pairs, 1.0 / 1e6 ** (2 * i / hd), 0.0).astype(np.float32)
    qkv_d = _t(qkv, dev)
    if nkv:
        kd = torch.zeros((nkv, max_ctx, hd), dtype=torch.float16, device=dev)
        vd = torch.zeros_like(kd)
        ops.qk_norm_rope_kv(qkv_d, kd, vd, _t(qw, dev), _t(kw, dev), _t(invf, dev), nh, pairs, 1e-6, pos0=pos)
    else:
        ops.qk_norm_rope_kv(qkv_d, None, None, _t(qw, dev), None, _t(invf, dev), nh, pairs, 1e-6, pos0=pos,
                            head_dim=hd)
    heads = qkv.reshape(nh + 2 * nkv, hd)
    q_want = np.stack([ref.rope(g4.rmsnorm_w(h, qw, 1e-6).astype(np.float32), pos, invf) for h in heads[:nh]])
    got = qkv_d.cpu().numpy().reshape(nh + 2 * nkv, hd)
    _close(got[:nh], q_want, 1e-5)
    if not nkv:
        assert np.array_equal(got[nh:], heads[nh:])
        return
    k_want = np.stack([ref.rope(g4.rmsnorm_w(h, kw, 1e-6).astype(np.float32), pos, invf)
                       for h in heads[nh:nh + nkv]]).astype(np.float16)
    v_want = np.stack([g4.rmsnorm_w(h, None, 1e-6) for h in heads[nh + nkv:]]).astype(np.float32).astype(np.float16)
    kg = _tile_rows(kd.cpu().numpy(), pos, "k").astype(np.float64)
    vg = _tile_rows(vd.cpu().numpy(), pos, "v").astype(np.float64)
    # fp16 of fp32 values: one fp16 ulp for the sin/cos and rsqrt rounding
    for g, w in ((kg, k_want), (vg, v_want)):
        w = w.astype(np.float64)
        assert np.max(np.abs(g - w) / np.maximum(np.abs(w), 6e-5)) <= 2 ** -10
    assert np.count_nonzero(kd.cpu().numpy()) == np.count_nonzero(k_want)


def _attn_case(rng, nh, nkv, hd, L, max_ctx):
    q = rng.standard_normal(nh * hd, dtype=np.float32) / math.sqrt(hd) * 4
    kc = np.zeros((nkv, max_ctx, hd), np.float16)
    vc = np.zeros((nkv, max_ctx, hd), np.float16)
    kc[:, :L] = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
    vc[:, :L] = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
    return q, kc, vc


def _window_ref(q, kc, vc, L, nh, window, scale=1.0):
    start = max(0, L - window) if window else 0
    return ref.attention(q, kc[:, start:L], vc[:, start:L], L - start, nh, scale)


@pytest.mark.parametrize("nh,nkv,hd", [(8, 1, 256), (8, 1, 512), (4, 1, 64), (8, 2, 128)])
@pytest.mark.parametrize("L,window", [(1, 16), (16, 16), (17, 16), (40, 16), (600, 512), (1000, 512),
                                      (4096, 512), (3000, 0), (33, 0)])
def test_attention_window(dev, rng, nh, nkv, hd, L, window):
    ops = _ops()
    max_ctx = max(64, (L + 31) // 32 * 32)
    q, kc, vc = _attn_case(rng, nh, nkv, hd, L, max_ctx)
    qd, kd, vd = _t(q, dev), _t(ops.to_tiles(kc, "k"), dev), _t(ops.to_tiles(vc, "v"), dev)
    out = ops.attention(qd, kd, vd, L, nh, scale=1.0, window=window)
    _close(out.cpu().numpy(), _window_ref(q, kc, vc, L, nh, window), 1e-3)
    # the position read on the device gives the same keys
    pos = torch.tensor([L - 1], dtype=torch.int32, device=dev)
    out2 = ops.attention(qd, kd, vd, 0, nh, scale=1.0, window=window, pos_dev=pos)
    assert torch.equal(out, out2)


def test_attention_window_ignores_keys_before_start(dev, rng):
    """Keys before the window start hold NaN/inf garbage; they must not leak in."""
    ops = _ops()
    nh, nkv, hd, L, window, max_ctx = 8, 1, 256, 100, 40, 128
    q, kc, vc = _attn_case(rng, nh, nkv, hd, L, max_ctx)
    kg, vg = kc.copy(), vc.copy()
    kg[:, : L - window] = np.float16(np.nan)
    vg[:, : L - window] = np.float16(np.inf)
    out = ops.attention(_t(q, dev), _t(ops.to_tiles(kg, "k"), dev), _t(ops.to_tiles(vg, "v"), dev), L, nh,
                        scale=1.0, window=window)
    _close(out.cpu().numpy(), _window_ref(q, kc, vc, L, nh, window), 1e-3)


@pytest.mark.parametrize("nh,hd", [(8, 256), (8, 512), (4, 64)])
@pytest.mark.parametrize("L,window,S", [(40, 16, 2), (300, 160, 2), (600, 512, 5), (1000, 512, 8), (200, 0, 3),
                                        (1, 512, 4)])
def test_attention_split_window_merged_by_o_projection(dev, rng, nh, hd, L, window, S):
    """The windowed split attention's partials (blocks dealt from the
    window's first block) merged by the o projection as it loads them: Wo .
    attention over the last `window` keys; the key count read on the device
    gives the same result."""
    ops = _ops()
    M, max_ctx = 512, max(64, (L + 31) // 32 * 32)
    q, kc, vc = _attn_case(rng, nh, 1, hd, L, max_ctx)
    Wo = (rng.standard_normal((M, nh * hd), dtype=np.float32) * 0.02).astype(np.float16)
    qd, kd, vd, wd = _t(q, dev), _t(ops.to_tiles(kc, "k"), dev), _t(ops.to_tiles(vc, "v"), dev), _t(Wo, dev)
    part = ops.attention_split(qd, kd, vd, L, nh, S, scale=1.0, window=window)
    got = ops.matvec_f16_attn_merge(wd, part, S, nh, hd, max_ctx, L, window=window).cpu().numpy()
    _close(got, ref.matvec(Wo, _window_ref(q, kc, vc, L, nh, window)), 1e-3)
    pos = torch.tensor([L - 1], dtype=torch.int32, device=dev)
    part2 = ops.attention_split(qd, kd, vd, 0, nh, S, scale=1.0, window=window, pos_dev=pos)
    got2 = ops.matvec_f16_attn_merge(wd, part2, S, nh, hd, max_ctx, 0, window=window, pos_dev=pos).cpu().numpy()
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("hd,window", [(128, 16), (512, 0), (256, 48)])
def test_attention_prefill_window(dev, rng, hd, window):
    ops = _ops()
    nh, nkv, pos0, rows, max_ctx = 4, 1, 37, 30, 128
    L = pos0 + rows
    q_rows = rng.standard_normal((rows, nh * hd), dtype=np.float32) / math.sqrt(hd) * 4
    _, kc, vc = _attn_case(rng, nh, nkv, hd, L, max_ctx)
    out = ops.attention_prefill(_t(q_rows, dev), _t(ops.to_tiles(kc, "k"), dev), _t(ops.to_tiles(vc, "v"), dev),
                                pos0, nh, scale=1.0, window=window).cpu().numpy()
    want = np.stack([_window_ref(q_rows[t], kc, vc, pos0 + t + 1, nh, window) for t in range(rows)])
    _close(out, want, 1e-3)


# ---------------------------------------------------------------- engine


@pytest.fixture(params=["folded", "separate"])
def g4_resadd(request):
    """The sandwich norms' residual adds folded into the next product (the
    default) or as their own launches (ENG_G4_RESADD=2)."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    _lib.set_tunable("ENG_G4_RESADD", 2 if request.param == "separate" else 1)
    try:
        yield request.param
    finally:
        _lib.set_tunable("ENG_G4_RESADD", 0)


def _shape(cfg: g4.G4Config):
    from gemmagemini4hackathon2026_10_2425_amd.engine import Gemma4Layer, Gemma4Shape

    layers = tuple(Gemma4Layer(y.head_dim, y.ffn_dim, y.sliding, y.kv_layer, y.rope_pairs, y.rope_theta,
                               y.layer_scalar) for y in cfg.layers)
    return Gemma4Shape(cfg.dim, cfg.n_heads, 1, cfg.vocab, cfg.ple_dim, cfg.ple_vocab, cfg.window, layers, cfg.eps,
                       cfg.softcap)


def _engine(cfg, max_ctx, seed, qk_norm_scale=1.0):
    """Engine with the synthetic weights; q/k norm weights scaled as the
    oracle's make_weights(qk_norm_scale) does (uploaded from it)."""
    from gemmagemini4hackathon2026_10_2425_amd.engine import Engine

    e = Engine(_shape(cfg), max_ctx)
    e.init_random(seed, 0.02)
    if qk_norm_scale != 1.0:
        w = g4.make_weights(cfg, seed, qk_norm_scale=qk_norm_scale)
        for name in w:
            if name.endswith(("q_norm", "k_norm")):
                e.upload(name, w[name])
    return e


def _golden():
    z = np.load(GOLDEN)
    return z, int(z["seed"]), float(z["qk_norm_scale"]), z["prompt"].tolist(), z["greedy"].tolist()


def test_gemma4_engine_weights_are_the_generator(dev):
    cfg = g4.G4_TINY
    want = g4.make_weights(cfg, 17)
    with _engine(cfg, 64, 17) as e:
        names = [n for n, _, _ in e.tensor_specs()]
        assert sorted(names) == sorted(want)
        for name, w in want.items():
            got = e.download(name, w.dtype).reshape(w.shape)
            assert np.array_equal(got.view(np.uint8), w.view(np.uint8)), name


def test_gemma4_engine_matches_oracle_every_position(dev, g4_resadd):
    """Softcapped logits after every step of prompt + greedy continuation, the
    positions past the sliding window (16) included."""
    cfg = g4.G4_TINY
    _, seed, qk, prompt, greedy = _golden()
    oracle = g4.G4Decoder(cfg, g4.make_weights(cfg, seed, qk_norm_scale=qk), 64)
    oracle.tokens[: len(prompt)] = prompt
    with _engine(cfg, 64, seed, qk) as e:
        e.set_tokens(prompt)
        for pos in range(len(prompt) + len(greedy) - 1):
            e.step(pos, sample=True)
            raw = oracle.forward(pos)
            _close(e.logits(), oracle.softcap(raw), 2e-3)
            if pos >= len(prompt) - 1:
                tok = ref.argmax(raw)
                oracle.tokens[pos + 1] = tok
                assert e.token(pos + 1) == tok, f"pos {pos}"
            else:
                e.set_tokens([prompt[pos + 1]], pos + 1)
        assert e.tokens(len(prompt), len(greedy)) == greedy


@pytest.mark.parametrize("fold", ["merged", "separate"])
def test_gemma4_engine_long_context_window(dev, fold):
    """A window of 160 keys at max_ctx 320: the sliding layers' attention runs
    as 2 splits whose partials the o projection merges (ENG_ATT_FOLD=2: the
    attention with its own output), the full layers as 3. A 250-token prompt
    stepped through the decode path (past the window), then 12 graph-replayed
    steps: the softcapped logits of the prompt's last position and of every
    replayed step within 2e-3 of the oracle, the same greedy tokens, and the
    replayed steps equal eager ones bit for bit."""
    import dataclasses

    from gemmagemini4hackathon2026_10_2425_amd import _lib

    cfg = dataclasses.replace(g4.G4_TINY, window=160)
    _, seed, qk, _, _ = _golden()
    prompt = np.random.default_rng(7).integers(0, cfg.vocab, 250).tolist()
    oracle = g4.G4Decoder(cfg, g4.make_weights(cfg, seed, qk_norm_scale=qk), 320)
    oracle.tokens[: len(prompt)] = prompt
    for pos in range(len(prompt)):
        raw = oracle.forward(pos)
    oracle.tokens[len(prompt)] = ref.argmax(raw)
    _lib.set_tunable("ENG_ATT_FOLD", 2 if fold == "separate" else 1)
    try:
        with _engine(cfg, 320, seed, qk) as a, _engine(cfg, 320, seed, qk) as b:
            _lib.set_tunable("ENG_NO_GEMM", 1)
            try:
                for e in (a, b):
                    e.set_tokens(prompt)
                    e.prefill(len(prompt))
            finally:
                _lib.set_tunable("ENG_NO_GEMM", 0)
            _close(a.logits(), oracle.softcap(raw), 2e-3)
            assert a.token(len(prompt)) == int(oracle.tokens[len(prompt)])
            for pos in range(len(prompt), len(prompt) + 12):
                raw = oracle.forward(pos)
                oracle.tokens[pos + 1] = ref.argmax(raw)
                a.decode(pos, 1)
                b.step(pos)
                got = a.logits()
                _close(got, oracle.softcap(raw), 2e-3)
                assert np.array_equal(got, b.logits()), f"pos {pos}: graph and eager steps differ"
            n = len(prompt)
            assert a.tokens(n, 13) == [int(t) for t in oracle.tokens[n : n + 13]]
            assert b.tokens(n, 13) == a.tokens(n, 13)
    finally:
        _lib.set_tunable("ENG_ATT_FOLD", 0)


def test_gemma4_engine_generate_matches_transformers(dev):
    """Prefill (token by token) then the graph-replayed decode: the greedy
    tokens of transformers' Gemma4ForCausalLM."""
    cfg = g4.G4_TINY
    _, seed, qk, prompt, greedy = _golden()
    with _engine(cfg, 64, seed, qk) as e:
        assert e.generate(prompt, len(greedy)) == greedy


def test_gemma4_engine_prefill_logits(dev):
    """The last prompt position's softcapped logits. The batched prefill rounds
    the activations entering each product to fp16 where the reference's chunk
    does: within 2e-3 of the oracle run the same way, and within the 1e-2
    contract of transformers (fp64). Token by token (ENG_NO_GEMM, the
    reference's --no-gemm) it is the decode path: within 2e-3 of transformers."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    cfg = g4.G4_TINY
    gold, seed, qk, prompt, _ = _golden()
    oracle = g4.G4Decoder(cfg, g4.make_weights(cfg, seed, qk_norm_scale=qk), 64)
    oracle.tokens[: len(prompt)] = prompt
    for pos in range(len(prompt)):
        want = oracle.softcap(oracle.forward(pos, half_acts=True))
    with _engine(cfg, 64, seed, qk) as e:
        e.set_tokens(prompt)
        e.prefill(len(prompt))
        _close(e.logits(), want, 2e-3)
        _close(e.logits(), gold["logits"][-1], 1e-2)
        _lib.set_tunable("ENG_NO_GEMM", 1)
        try:
            e.set_tokens(prompt)
            e.prefill(len(prompt))
        finally:
            _lib.set_tunable("ENG_NO_GEMM", 0)
        _close(e.logits(), gold["logits"][-1], 2e-3)


@pytest.mark.parametrize("chunk", [256, 0], ids=["chunk256", "default-chunk"])
def test_gemma4_engine_prefill_chunks(dev, chunk):
    """A prompt of 300 rows, far past the window of 16, as two chunks (256 +
    44 rows: the second attends to the first's cached keys) and as one (the
    default 1024-row chunk); the last row's logits match the oracle run with
    the prefill's fp16 activation points."""
    from gemmagemini4hackathon2026_10_2425_amd import _lib

    cfg = g4.G4_TINY
    _, seed, qk, _, _ = _golden()
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 300).tolist()
    oracle = g4.G4Decoder(cfg, g4.make_weights(cfg, seed, qk_norm_scale=qk), 320)
    oracle.tokens[: len(prompt)] = prompt
    for pos in range(len(prompt)):
        raw = oracle.forward(pos, half_acts=True)
    _lib.set_tunable("ENG_PREFILL_ROWS", chunk)
    try:
        with _engine(cfg, 320, seed, qk) as e:
            e.set_tokens(prompt)
            e.prefill(len(prompt))
            _close(e.logits(), oracle.softcap(raw), 2e-3)
    finally:
        _lib.set_tunable("ENG_PREFILL_ROWS", 0)


def test_gemma4_engine_decode_graph_equals_steps(dev, g4_resadd):
    cfg = g4.G4_TINY
    prompt = [5, 17, 999, 3, 250]
    with _engine(cfg, 64, 3, 0.25) as a, _engine(cfg, 64, 3, 0.25) as b:
        a.set_tokens(prompt)
        a.prefill(len(prompt))
        a.decode(len(prompt), 40)
        b.set_tokens(prompt)
        b.prefill(len(prompt))
        for pos in range(len(prompt), len(prompt) + 40):
            b.step(pos)
        b.sync()
        assert a.tokens(len(prompt), 41) == b.tokens(len(prompt), 41)


# ---------------------------------------------------------------- weight file + CLI


@pytest.fixture(scope="module")
def g4_file(tmp_path_factory):
    """The golden checkpoint as a local multimodal-layout HF directory,
    converted to the reference's Gemma-4 file."""
    from gemmagemini4hackathon2026_10_2425_amd import weights
    from tests.test_gemma4_host import _g4_snapshot

    _, seed, qk, _, _ = _golden()
    d = tmp_path_factory.mktemp("g4")
    _g4_snapshot(d / "snap", g4.G4_TINY, g4.make_weights(g4.G4_TINY, seed, qk_norm_scale=qk), multimodal=True)
    weights.convert_hf(d / "snap", d / "g4.bin")
    return d / "g4.bin"


def test_gemma4_load_engine_matches_transformers(dev, g4_file):
    from gemmagemini4hackathon2026_10_2425_amd.weights import load_engine

    gold, _, _, prompt, greedy = _golden()
    with load_engine(g4_file, 64) as e:
        assert e.generate(prompt, len(greedy)) == greedy
        e.set_tokens(prompt)
        e.prefill(len(prompt))
        _close(e.logits(), gold["logits"][-1], 1e-2)


def test_gemma4_cli_generate_and_dump_logits(dev, g4_file, tmp_path):
    """The engine binary on the Gemma-4 file: greedy ids and the softcapped
    --dump-logits (KG/main.swift:657-662) against transformers."""
    import json
    import os
    import subprocess
    import sys

    gold, _, _, prompt, greedy = _golden()
    root = Path(__file__).resolve().parents[1]
    p = subprocess.run([sys.executable, "-m", "gemmagemini4hackathon2026_10_2425_amd.serve", "--weights", str(g4_file),
                        "--max-ctx", "64", "--prompt-ids", ",".join(map(str, prompt)), "--gen", str(len(greedy)),
                        "--dump-logits", str(tmp_path / "l.f32")], capture_output=True, text=True, timeout=240,
                       cwd=root, env=dict(os.environ))
    assert p.returncode == 0, p.stderr[-2000:]
    assert json.loads(p.stdout.strip().splitlines()[-1])["tokens"] == greedy
    logits = np.fromfile(tmp_path / "l.f32", "<f4")
    assert logits.shape == (g4.G4_TINY.vocab,) and np.abs(logits).max() < g4.G4_TINY.softcap
    _close(logits, gold["logits"][-1], 1e-2)
