"""Pins for the CPU oracle (runs without a GPU).

The reference has no per-operator tests or golden vectors (its only checks are
end-to-end strings on real checkpoints, ios_kernels/surfaces/tests/
test_kernel_e2e.py:23-32). Each oracle function is pinned here instead by
something independent of its own formula: a closed form, a library routine
(torch / transformers), brute force, a second restatement (the C oracle), or
HF transformers' Gemma on a tiny config (tests/golden/hf_gemma_tiny.npz).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import batch as ob, hashrng, model as om, native, ops

# ---------------------------------------------------------------- generator


def test_hashrng_three_restatements_agree():
    v = hashrng.normal_f32(64, 1234, 1000 + 16 * 3 + 4, 0.02)
    ints = [hashrng.normal_int(i, 1234, 1000 + 16 * 3 + 4, 0.02) for i in range(64)]
    assert np.array_equal(v, np.array(ints, np.float32))
    c = native.fill_normal((64,), np.float32, 1234, 1000 + 16 * 3 + 4, 0.02)
    assert np.array_equal(v, c)
    h_np = hashrng.normal((50000,), np.float16, 9, 1, 0.02)
    h_c = native.fill_normal((50000,), np.float16, 9, 1, 0.02)
    assert np.array_equal(h_np.view(np.uint16), h_c.view(np.uint16))


def test_hashrng_mix_is_splitmix64():
    # splitmix64 from state 0: first outputs of the published generator.
    assert hashrng.mix_int(0) == 0xE220A8397B1DCDAF
    assert hashrng.mix_int(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    z = np.array([0, 0x9E3779B97F4A7C15], np.uint64)
    assert hashrng.mix(z).tolist() == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]


def test_hashrng_statistics():
    v = hashrng.normal_f32(1 << 20, 5, 77, 1.0).astype(np.float64)
    assert abs(v.mean()) < 5e-3
    assert abs(v.std() - 1.0) < 5e-3
    kurt = ((v - v.mean()) ** 4).mean() / v.var() ** 2
    assert abs(kurt - (3 - 1.2 / 8)) < 0.03  # Irwin-Hall(8): excess kurtosis -6/(5*8)
    assert np.abs(v).max() <= 4 * 65535 / hashrng.SIGMA_SUM + 1e-6
    w = hashrng.normal_f32(1 << 16, 5, 78, 0.02)
    assert abs(w.std() - 0.02) < 5e-4
    assert not np.array_equal(hashrng.normal_f32(16, 5, 77, 1.0), hashrng.normal_f32(16, 5, 79, 1.0))


# ---------------------------------------------------------------- matvec


def test_matvec_closed_forms(rng):
    x = rng.standard_normal(64)
    assert np.array_equal(ops.matvec(np.eye(64, dtype=np.float16), x), x)
    W = rng.standard_normal((5, 64)).astype(np.float16)
    assert np.array_equal(ops.matvec(W, np.eye(64)[7]), W[:, 7].astype(np.float64))
    assert np.allclose(ops.matvec(np.ones((3, 64), np.float16), x), x.sum())


def test_matvec_brute_force(rng):
    W = rng.standard_normal((7, 40)).astype(np.float16)
    x = rng.standard_normal(40).astype(np.float32)
    brute = [math.fsum(float(W[r, k]) * float(x[k]) for k in range(40)) for r in range(7)]
    assert np.allclose(ops.matvec(W, x), brute, rtol=0, atol=1e-12)
    assert np.allclose(native.matvec_f16(W, x), brute, rtol=0, atol=1e-12)


def test_matvec_linearity(rng):
    W = rng.standard_normal((9, 32)).astype(np.float16)
    a, b = rng.standard_normal(32), rng.standard_normal(32)
    assert np.allclose(ops.matvec(W, 2 * a - 3 * b), 2 * ops.matvec(W, a) - 3 * ops.matvec(W, b))


def test_quantize_closed_forms():
    s = np.float16(0.5)
    W = np.zeros((3, 64), np.float32)
    W[0, :32] = np.arange(-16, 16) * float(s)  # exact multiples of s with max 16*s -> s' = 16s/127
    W[1, :32] = 127 * float(s)                  # a block at +127 s
    W[1, 32:] = -127 * float(s)
    q, sc = ops.quantize_q8b32(W)
    assert sc[2, 0] == 0 and sc[2, 1] == 0 and not q[2].any()  # zero blocks
    assert sc[1, 0] == s and np.all(q[1, :32] == 127) and np.all(q[1, 32:] == -127)
    deq = q.astype(np.float32).reshape(3, 2, 32) * sc.astype(np.float32)[..., None]
    assert np.array_equal(deq[1].reshape(-1), W[1])


def test_quantize_roundtrip_and_package_agree(rng):
    from gemmagemini4hackathon2026_10_2425_amd.quant import quantize_q8b32

    W = rng.standard_normal((33, 320)).astype(np.float32) * 0.02
    W[4, 32:64] = 0.0
    q, s = ops.quantize_q8b32(W)
    q2, s2 = quantize_q8b32(W)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint16), s2.view(np.uint16))
    deq = q.reshape(33, 10, 32).astype(np.float64) * s.astype(np.float64)[..., None]
    err = np.abs(deq.reshape(33, 320) - W)
    bound = (s.astype(np.float64)[..., None] * np.ones((1, 1, 32))).reshape(33, 320) * 0.5
    # fp16 rounding of the scale adds up to 127 * s * 2^-11 on top of s/2
    assert np.all(err <= bound * (1 + 127 * 2**-10) + 1e-12)
    assert np.abs(q).max() <= 127


def test_matvec_q8b32_equals_dequant(rng):
    W = rng.standard_normal((17, 256)).astype(np.float32)
    q, s = ops.quantize_q8b32(W)
    x = rng.standard_normal(256).astype(np.float32)
    deq = q.reshape(17, 8, 32).astype(np.float64) * s.astype(np.float64)[..., None]
    assert np.allclose(ops.matvec_q8b32(q, s, x), deq.reshape(17, 256) @ x, rtol=1e-13, atol=1e-13)
    assert np.allclose(native.matvec_q8b32(q, s, x), ops.matvec_q8b32(q, s, x), rtol=1e-13, atol=1e-13)


# ---------------------------------------------------------------- activations


def test_activations_match_torch(rng):
    g = torch.from_numpy(rng.standard_normal(1000) * 6)
    want_gelu = torch.nn.functional.gelu(g, approximate="tanh").numpy()
    assert np.allclose(ops.gelu_tanh(g.numpy()), want_gelu, rtol=1e-13, atol=1e-15)
    assert np.allclose(ops.silu(g.numpy()), torch.nn.functional.silu(g).numpy(), rtol=1e-13, atol=1e-15)
    assert ops.gelu_tanh(0.0) == 0.0 and ops.silu(0.0) == 0.0
    assert abs(ops.gelu_tanh(30.0) - 30.0) < 1e-12 and abs(ops.silu(40.0) - 40.0) < 1e-12


def test_gate_up_special_cases(rng):
    Wg = np.zeros((4, 32), np.float16)
    Wu = rng.standard_normal((4, 32)).astype(np.float16)
    x = rng.standard_normal(32)
    assert np.all(ops.gate_up(Wg, Wu, x) == 0)


# ---------------------------------------------------------------- rmsnorm


def test_rmsnorm_matches_torch(rng):
    x = rng.standard_normal((3, 2048)) * 5
    w = rng.standard_normal(2048) * 0.02
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (2048,), torch.from_numpy(w), eps=1e-6).numpy()
    assert np.allclose(ops.rmsnorm(x, w, 1e-6), want, rtol=1e-12, atol=1e-14)
    want1 = torch.nn.functional.rms_norm(torch.from_numpy(x), (2048,), torch.from_numpy(1 + w), eps=1e-6).numpy()
    assert np.allclose(ops.rmsnorm(x, w, 1e-6, plus_one=True), want1, rtol=1e-12, atol=1e-14)


def test_rmsnorm_closed_forms():
    c, eps = 3.0, 1e-6
    y = ops.rmsnorm(np.full(16, c), np.full(16, 2.0), eps)
    assert np.allclose(y, c / math.sqrt(c * c + eps) * 2.0)
    x = np.arange(1, 9, dtype=np.float64)
    assert np.allclose(ops.rmsnorm(x * 1000, np.ones(8), 0.0), ops.rmsnorm(x, np.ones(8), 0.0))


# ---------------------------------------------------------------- rope


def test_rope_identity_and_norm(rng):
    invf = ops.inv_freq(128, 10000.0)
    v = rng.standard_normal(128)
    assert np.allclose(ops.rope(v, 0, invf), v)
    r = ops.rope(v, 777, invf)
    pn = lambda a: a[:64] ** 2 + a[64:] ** 2  # noqa: E731
    assert np.allclose(pn(r), pn(v))


def test_rope_composition():
    # inv_freq of powers of two keeps fp32 angles exact, so R(a) R(b) = R(a + b).
    invf = np.array([2.0 ** -k for k in range(64)], np.float32)
    v = np.random.default_rng(1).standard_normal(128)
    assert np.allclose(ops.rope(ops.rope(v, 5, invf), 9, invf), ops.rope(v, 14, invf), atol=1e-12)


def test_rope_matches_hf_apply_rotary():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    rng = np.random.default_rng(3)
    hd, pos = 256, 300
    invf = ops.inv_freq(hd, 10000.0)
    q = rng.standard_normal((1, 2, 1, hd))
    k = rng.standard_normal((1, 1, 1, hd))
    ang = (np.float32(pos) * invf).astype(np.float64)
    emb = np.concatenate([ang, ang])
    cos, sin = torch.from_numpy(np.cos(emb))[None, None], torch.from_numpy(np.sin(emb))[None, None]
    qh, kh = apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(k), cos, sin, unsqueeze_dim=1)
    assert np.allclose(ops.rope(q[0, :, 0], pos, invf), qh.numpy()[0, :, 0], atol=1e-12)
    assert np.allclose(ops.rope(k[0, :, 0], pos, invf), kh.numpy()[0, :, 0], atol=1e-12)


def test_inv_freq_definition():
    f = ops.inv_freq(128, 500000.0)
    assert f[0] == 1.0 and f.dtype == np.float32
    assert f[63] == np.float32(1.0 / 500000.0 ** (126 / 128))


def test_inv_freq_llama3_matches_hf():
    """Llama-3 frequency scaling (Llama-3.2-1B's rope_scaling) against
    transformers' llama3 rope initialiser (fp32); the Llama-3.2-1B head_dim 64
    puts frequencies in all three bands (kept, divided, blended)."""
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    rp = {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 32.0, "low_freq_factor": 1.0,
          "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    hc = LlamaConfig(hidden_size=2048, num_attention_heads=32, head_dim=64, max_position_embeddings=131072,
                     rope_parameters=rp)
    want, _ = ROPE_INIT_FUNCTIONS["llama3"](hc, "cpu")
    got = ops.inv_freq_llama3(64, 500000.0, 32.0, 1.0, 4.0, 8192)
    assert got.dtype == np.float32
    assert np.abs(want.numpy().astype(np.float64) / got - 1).max() < 1e-6
    base = ops.inv_freq(64, 500000.0)
    kept, divided = got == base, np.isclose(got, base / 32, rtol=1e-7)
    assert kept.sum() >= 8 and divided.sum() >= 8 and (~kept & ~divided).sum() >= 2
    assert np.all(np.diff(got) < 0)  # still strictly decreasing


def test_rope_kv_appends_fp16(rng):
    nh, nkv, hd, ctx = 4, 2, 128, 16
    kc = np.zeros((nkv, ctx, hd), np.float16)
    vc = np.zeros((nkv, ctx, hd), np.float16)
    row = rng.standard_normal((nh + 2 * nkv) * hd).astype(np.float32)
    invf = ops.inv_freq(hd, 10000.0)
    q = ops.rope_kv(row, kc, vc, invf, nh, nkv, 5)
    assert np.allclose(q.reshape(nh, hd), ops.rope(row[: nh * hd].reshape(nh, hd), 5, invf))
    k_want = ops.rope(row[nh * hd : (nh + nkv) * hd].reshape(nkv, hd), 5, invf).astype(np.float16)
    assert np.array_equal(kc[:, 5, :], k_want)
    assert np.array_equal(vc[:, 5, :], row[(nh + nkv) * hd :].reshape(nkv, hd).astype(np.float16))
    assert np.count_nonzero(kc[:, :5]) == 0 and np.count_nonzero(vc[:, 6:]) == 0


# ---------------------------------------------------------------- attention


def _cache(rng, nkv, L, hd):
    K = rng.standard_normal((nkv, L, hd)).astype(np.float16)
    V = rng.standard_normal((nkv, L, hd)).astype(np.float16)
    return K, V, V


def test_attention_matches_torch_sdpa(rng):
    nh, nkv, hd, L = 8, 2, 128, 50
    K, Vt, V = _cache(rng, nkv, L, hd)
    q = rng.standard_normal(nh * hd)
    got = ops.attention(q, K, Vt, L, nh, 1 / math.sqrt(hd))
    G = nh // nkv
    Kr = torch.from_numpy(K.astype(np.float64)).repeat_interleave(G, 0)[None]
    Vr = torch.from_numpy(V.astype(np.float64)).repeat_interleave(G, 0)[None]
    qt = torch.from_numpy(q.reshape(1, nh, 1, hd))
    want = torch.nn.functional.scaled_dot_product_attention(qt, Kr, Vr, scale=1 / math.sqrt(hd)).numpy()
    assert np.allclose(got, want.reshape(-1), rtol=1e-12, atol=1e-13)


def test_attention_closed_forms(rng):
    nh, nkv, hd = 4, 1, 128
    K, Vt, V = _cache(rng, nkv, 10, hd)
    q = rng.standard_normal(nh * hd)
    one = ops.attention(q, K, Vt, 1, nh, 0.1).reshape(nh, hd)
    assert np.allclose(one, np.broadcast_to(V[0, 0].astype(np.float64), (nh, hd)))
    Ks = np.broadcast_to(K[:, :1], K.shape).copy()
    same = ops.attention(q, Ks, Vt, 10, nh, 0.1).reshape(nh, hd)
    assert np.allclose(same, V[0].astype(np.float64).mean(axis=0))
    # a constant shift of all scores (q orthogonal part) does not change the output
    K2 = K.astype(np.float64) + 0.0
    a = ops.attention(q, K2, Vt, 10, nh, 0.1)
    assert np.allclose(a, ops.attention(q, K, Vt, 10, nh, 0.1))


def test_attention_split_merge_identity(rng):
    """The log-sum-exp merge the GPU uses equals one pass (the rule itself, in fp64)."""
    nh, nkv, hd, L = 2, 1, 128, 96
    K, Vt, _ = _cache(rng, nkv, L, hd)
    q = rng.standard_normal(nh * hd)
    s = (K[0].astype(np.float64) @ q.reshape(nh, hd).T).T * 0.2  # [nh, L]
    V = Vt[0].astype(np.float64)
    parts = []
    for a, b in [(0, 30), (30, 64), (64, 96)]:
        m = s[:, a:b].max(axis=1, keepdims=True)
        p = np.exp(s[:, a:b] - m)
        parts.append((m, p.sum(axis=1, keepdims=True), p @ V[a:b]))
    M = np.max([m for m, _, _ in parts], axis=0)
    num = sum(np.exp(m - M) * o for m, _, o in parts)
    den = sum(np.exp(m - M) * l for m, l, _ in parts)
    assert np.allclose(num / den, ops.attention(q, K, Vt, L, nh, 0.2).reshape(nh, hd))


def test_argmax_first_max():
    x = np.array([1.0, 5.0, 2.0, 5.0, -1.0], np.float32)
    assert ops.argmax(x) == 1
    assert ops.argmax(np.zeros(10, np.float32)) == 0


def _argmax_scan(v) -> int:
    """The reference's loop, literally: best = -inf, index 0, take v > best."""
    best, idx = -math.inf, 0
    for i, x in enumerate(v):
        if x > best:
            best, idx = float(x), i
    return idx


def test_argmax_nan_and_inf_like_the_reference_scan(rng):
    nan, inf = np.float32("nan"), np.float32("inf")
    cases = [np.array([nan, 1.0, 3.0, nan], np.float32), np.array([nan, nan], np.float32),
             np.array([-inf, nan, -inf], np.float32), np.array([2.0, inf, nan, inf], np.float32),
             np.array([-inf, -5.0], np.float32)]
    for _ in range(50):
        v = rng.standard_normal(40).astype(np.float32)
        v[rng.random(40) < 0.2] = nan
        v[rng.random(40) < 0.1] = -inf
        v[rng.random(40) < 0.05] = inf
        cases.append(v)
    for v in cases:
        assert ops.argmax(v) == _argmax_scan(v), v
    assert ops.argmax(cases[0]) == 2 and ops.argmax(cases[1]) == 0 and ops.argmax(cases[2]) == 0


def test_embed_closed_form(rng):
    E = rng.standard_normal((10, 8)).astype(np.float16)
    assert np.array_equal(ops.embed(E, 3, 2.0), E[3].astype(np.float64) * 2.0)


# ---------------------------------------------------------------- decode step


def test_decode_matches_hf_gemma():
    """Logits of every prompt position and the greedy continuation equal HF
    transformers' GemmaForCausalLM (fp64) on the same weights."""
    z = np.load(__file__.rsplit("/", 1)[0] + "/golden/hf_gemma_tiny.npz")
    cfg = om.TINY
    d = om.OracleDecoder(cfg, om.make_weights(cfg, int(z["seed"]), float(z["std"]), float(z["embed_std"])), 64,
                         fp16_kv=False)
    prompt = [int(t) for t in z["prompt"]]
    d.tokens[: len(prompt)] = prompt
    for pos in range(len(prompt)):
        lg = d.forward(pos)
        ref = z["logits"][pos]
        assert np.abs(lg - ref).max() / np.abs(ref).max() < 1e-6
    toks, _ = d.generate(prompt, len(z["greedy"]))
    assert toks == [int(t) for t in z["greedy"]]


def test_prefill_chunk_pins():
    """The batched prefill restatement: without its fp16 activation roundings
    every row's logits equal the token-by-token path's (pinned to HF above);
    chunking the prompt changes nothing; with the roundings the last row stays
    within the 1e-2 contract of HF's logits and gives HF's first greedy token."""
    z = np.load(__file__.rsplit("/", 1)[0] + "/golden/hf_gemma_tiny.npz")
    cfg = om.TINY
    w = om.make_weights(cfg, int(z["seed"]), float(z["std"]), float(z["embed_std"]))
    prompt = [int(t) for t in z["prompt"]]
    P = len(prompt)
    for rows in range(1, P + 1):
        a = om.OracleDecoder(cfg, w, 64)
        a.tokens[:P] = prompt
        lg = a.prefill_chunk(0, rows, half_acts=False)
        b = om.OracleDecoder(cfg, w, 64)
        b.tokens[:P] = prompt
        for pos in range(rows):
            want = b.forward(pos)
        assert np.abs(lg - want).max() / np.abs(want).max() < 1e-5, rows
        assert np.array_equal(a.k, b.k) and np.array_equal(a.v, b.v), rows
    whole = om.OracleDecoder(cfg, w, 64)
    whole.tokens[:P] = prompt
    lg_whole = whole.prefill_chunk(0, P)
    parts = om.OracleDecoder(cfg, w, 64)
    parts.tokens[:P] = prompt
    parts.prefill_chunk(0, 3, sample=False)
    lg_parts = parts.prefill_chunk(3, P - 3)
    assert np.array_equal(lg_whole, lg_parts) and np.array_equal(whole.k, parts.k)
    assert np.abs(lg_whole - z["logits"][P - 1]).max() / np.abs(z["logits"][P - 1]).max() < 1e-2
    assert int(whole.tokens[P]) == int(z["greedy"][0])


_C_VS_NUMPY = [
    (om.DecodeConfig(n_layers=2, dim=256, n_heads=8, n_kv_heads=1, head_dim=256, ffn_dim=512, vocab=2000), None),
    # Llama-3.2-1B features: head_dim 64, GQA, Llama-3 RoPE scaling, untied lm_head
    (om.DecodeConfig(n_layers=2, dim=256, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=2000, eps=1e-5,
                     rope_theta=500000.0, act="silu", gemma_embed_scale=False, plus_one=False, tie_embeddings=False,
                     rope_scaling=(32.0, 1.0, 4.0, 8192)), None),
    # the embedding at its own scale
    (om.DecodeConfig(n_layers=2, dim=256, n_heads=8, n_kv_heads=1, head_dim=256, ffn_dim=512, vocab=2000), 0.005),
]


@pytest.mark.parametrize("cfg,embed_std", _C_VS_NUMPY, ids=["gemma-mqa256", "llama32-hd64-untied", "embed-std"])
def test_decode_numpy_and_c_restatements_agree(cfg, embed_std):
    seed = 21
    d = om.OracleDecoder(cfg, om.make_weights(cfg, seed, embed_std=embed_std), 64)
    n = native.NativeDecoder(cfg, 64, seed, embed_std=embed_std)
    assert np.array_equal(n.inv_freq(), d.invf)
    prompt = [7, 1999, 0, 1234, 55]
    t1, m1 = d.generate(prompt, 10)
    t2, m2 = n.generate(prompt, 10)
    assert t1 == t2
    assert np.allclose(m1, m2, rtol=1e-4, atol=1e-5)
    d2 = om.OracleDecoder(cfg, om.make_weights(cfg, seed, embed_std=embed_std), 64)
    d2.tokens[: len(prompt)] = prompt
    n2 = native.NativeDecoder(cfg, 64, seed, embed_std=embed_std)
    n2.tokens[: len(prompt)] = prompt
    for pos in range(len(prompt)):
        a = d2.forward(pos)
        _, _, b = n2.step(pos, want_logits=True, sample=False)
        assert np.abs(a - b).max() / np.abs(a).max() < 1e-5


@pytest.mark.parametrize("name", ["embed", "final_norm", "l0.attn_norm", "l17.wdown"])
def test_tensor_ids_are_distinct(name):
    ids = {om.tensor_id(n) for n in om.weight_shapes(om.GEMMA_2B)}
    assert len(ids) == len(om.weight_shapes(om.GEMMA_2B))
    assert om.tensor_id(name) in ids


# ---------------------------------------------------------------- ragged-batch layer (oracle.batch)


def test_batch_dequant_closed_forms():
    q = np.zeros((2, 64), np.int8)
    q[0, :32] = np.arange(-16, 16)
    q[1, 32:] = -127
    s = np.array([[0.5, 3.0], [2.0, 0.25]], np.float16)
    d = ob.dequant(q, s)
    assert np.array_equal(d[0, :32], np.arange(-16, 16) * 0.5) and not d[0, 32:].any()
    assert not d[1, :32].any() and np.all(d[1, 32:] == -127 * 0.25)


def test_batch_dequant_f16_rounds_each_weight(rng):
    """The fp16-weight mode: every weight within half an fp16 ulp of q * s
    (relative 2^-11 for normal values), exact where q * s is representable
    (q * 2^k, |q| <= 127 < 2^11), and a product of it is within
    2^-11 * sum |w x| of the exact one."""
    q = rng.integers(-127, 128, (40, 256)).astype(np.int8)
    s = (np.abs(rng.standard_normal((40, 8))) * 1e-3 + 1e-4).astype(np.float16)
    exact, rounded = ob.dequant(q, s), ob.dequant(q, s, f16=True)
    nz = exact != 0
    assert np.all(np.abs(rounded - exact)[nz] <= np.abs(exact)[nz] * 2.0**-11)
    pow2 = np.full((1, 8), 0.0078125, np.float16)  # 2^-7: every product exact in fp16
    assert np.array_equal(ob.dequant(q[:1], pow2, f16=True), ob.dequant(q[:1], pow2))
    X = rng.standard_normal((5, 256)).astype(np.float16)
    d = ob.gemm_q8b32(q, s, X, True) - ob.gemm_q8b32(q, s, X)
    bound = 2.0**-11 * (np.abs(X.astype(np.float64)) @ np.abs(exact).T)
    assert np.all(np.abs(d) <= bound * (1 + 1e-9))


def test_batch_gemm_q8b32_rows_equal_matvec(rng):
    W = rng.standard_normal((23, 320)).astype(np.float32) * 0.02
    q, s = ops.quantize_q8b32(W)
    X = rng.standard_normal((5, 320)).astype(np.float16)
    Y = ob.gemm_q8b32(q, s, X)
    assert Y.shape == (5, 23)
    for b in range(5):
        assert np.allclose(Y[b], ops.matvec_q8b32(q, s, X[b]), rtol=1e-13, atol=1e-15), b


def test_batch_gemm_q8b32_brute_force(rng):
    q = rng.integers(-127, 128, (3, 64)).astype(np.int8)
    s = (rng.random((3, 2)) * 0.01).astype(np.float16)
    X = rng.standard_normal((2, 64)).astype(np.float32)
    want = [[math.fsum(float(q[r, k]) * float(s[r, k // 32]) * float(X[b, k]) for k in range(64)) for r in range(3)]
            for b in range(2)]
    assert np.allclose(ob.gemm_q8b32(q, s, X), want, rtol=0, atol=1e-15)


def test_batch_gate_up_rows_equal_per_row(rng):
    qg, sg = ops.quantize_q8b32(rng.standard_normal((16, 96)).astype(np.float32) * 0.05)
    qu, su = ops.quantize_q8b32(rng.standard_normal((16, 96)).astype(np.float32) * 0.05)
    X = rng.standard_normal((4, 96)).astype(np.float16)
    for act in ("silu", "gelu_tanh"):
        H = ob.gate_up_rows(qg, sg, qu, su, X, act)
        for b in range(4):
            want = ops.gate_up_q8b32(qg, sg, qu, su, X[b], act)
            assert np.allclose(H[b], want, rtol=1e-12, atol=1e-15), (act, b)
    assert not ob.gate_up_rows(np.zeros_like(qg), sg, qu, su, X, "silu").any()  # act(0) = 0


def _hf_layer_fixture():
    z = np.load(Path(__file__).resolve().parent / "golden" / "hf_llama_layer.npz")
    D, NH, NKV, HD, F = (int(v) for v in z["dims"])
    cfg = ob.LayerConfig(D, NH, NKV, HD, F, eps=float(z["eps"]), rope_theta=float(z["rope_theta"]))
    seed = int(z["seed"])
    lens, starts = [int(v) for v in z["lens"]], [int(v) for v in z["starts"]]
    X = [hashrng.normal((n, D), np.float32, seed, 500 + b, 1.0) for b, n in enumerate(lens)]
    offs = np.concatenate([[0], np.cumsum(lens)])
    want = [z["out"][offs[b] : offs[b + 1]] for b in range(len(lens))]
    return cfg, ob.synthetic_layer(cfg, seed), lens, starts, X, want


def _stagger(cfg, W, lens, starts, X, half_acts, kv_dtype):
    """Steps every sequence token by token; sequence b joins the batch at step
    starts[b], so one batch holds sequences at different positions. Returns
    each sequence's output rows."""
    kc = [np.zeros((cfg.n_kv_heads, n, cfg.head_dim), kv_dtype) for n in lens]
    vc = [np.zeros((cfg.n_kv_heads, n, cfg.head_dim), kv_dtype) for n in lens]
    out = [np.zeros((n, cfg.dim), np.float32) for n in lens]
    for t in range(max(s + n for s, n in zip(starts, lens))):
        act = [b for b in range(len(lens)) if starts[b] <= t < starts[b] + lens[b]]
        pos = [t - starts[b] for b in act]
        Y = ob.layer_step(cfg, W, np.stack([X[b][p] for b, p in zip(act, pos)]), [kc[b] for b in act],
                          [vc[b] for b in act], np.array(pos) + 1, half_acts=half_acts)
        for i, (b, p) in enumerate(zip(act, pos)):
            out[b][p] = Y[i]
    return out


def test_batch_layer_step_matches_hf_llama_layer():
    """Without the fp16 activation roundings and with fp64 caches, every row of
    a staggered ragged batch equals transformers' LlamaDecoderLayer (float64)
    on the dequantised weights, up to the fp32 storage of each output."""
    cfg, W, lens, starts, X, want = _hf_layer_fixture()
    got = _stagger(cfg, W, lens, starts, X, half_acts=False, kv_dtype=np.float64)
    for b in range(len(lens)):
        assert np.abs(got[b] - want[b]).max() / np.abs(want[b]).max() < 1e-6, b
    # the device's roundings (fp16 activations and K/V) stay inside the 1e-2 contract
    got16 = _stagger(cfg, W, lens, starts, X, half_acts=True, kv_dtype=np.float16)
    for b in range(len(lens)):
        assert np.abs(got16[b] - want[b]).max() / np.abs(want[b]).max() < 3e-3, b


def test_batch_layer_step_ragged_equals_single_sequences():
    """A sequence's rows do not depend on which other sequences share its batch."""
    cfg, W, lens, starts, X, _ = _hf_layer_fixture()
    together = _stagger(cfg, W, lens, starts, X, half_acts=True, kv_dtype=np.float16)
    for b in range(len(lens)):
        alone = _stagger(cfg, W, [lens[b]], [0], [X[b]], half_acts=True, kv_dtype=np.float16)[0]
        assert np.allclose(together[b], alone, rtol=1e-6, atol=1e-7), b


# ---------------------------------------------------------------- Gemma-4 (oracle.gemma4)


def _g4_golden():
    from oracle import gemma4 as g4

    z = np.load(Path(__file__).resolve().parent / "golden" / "hf_gemma4_tiny.npz")
    return g4, z, [int(t) for t in z["prompt"]]


def test_gemma4_matches_hf_gemma4():
    """Every prompt position's logits (softcapped) equal transformers'
    Gemma4ForCausalLM in float64 on the same weights, up to the oracle's fp32
    storage between ops (K/V kept in fp64 here), and the greedy continuation
    with the device's fp16 K/V is HF's: sliding window, proportional RoPE, KV
    sharing, double-width MLPs, q/k/v norms, sandwich norms, per-layer
    embeddings and layer scalars are all in the tiny config."""
    g4, z, prompt = _g4_golden()
    cfg = g4.G4_TINY
    w = g4.make_weights(cfg, int(z["seed"]), qk_norm_scale=float(z["qk_norm_scale"]))
    d = g4.G4Decoder(cfg, w, 64, fp16_kv=False)
    d.tokens[: len(prompt)] = prompt
    for pos in range(len(prompt)):
        lg = d.softcap(d.forward(pos))
        ref = z["logits"][pos]
        assert np.abs(lg - ref).max() / np.abs(ref).max() < 2e-5, pos
    toks, margins = g4.G4Decoder(cfg, w, 64).generate(prompt, len(z["greedy"]))
    assert toks == [int(t) for t in z["greedy"]]
    assert len(set(toks)) >= 9  # not a run stuck on one token
    assert min(margins) > 0.01


def test_gemma4_half_activation_prefill():
    """The prefill mode (activations rounded to fp16 before each product, as
    the reference's chunk stores them) stays within the 1e-2 contract of
    transformers' fp64 logits, and does round: it moves the logits by more
    than fp32 storage alone does."""
    g4, z, prompt = _g4_golden()
    cfg = g4.G4_TINY
    w = g4.make_weights(cfg, int(z["seed"]), qk_norm_scale=float(z["qk_norm_scale"]))
    d = g4.G4Decoder(cfg, w, 64, fp16_kv=False)
    d.tokens[: len(prompt)] = prompt
    errs = []
    for pos in range(len(prompt)):
        ref = z["logits"][pos]
        errs.append(np.abs(d.softcap(d.forward(pos, half_acts=True)) - ref).max() / np.abs(ref).max())
    assert max(errs) < 1e-2 and max(errs) > 1e-4


def test_gemma4_e2b_layer_facts():
    """The E2B per-layer facts as the reference's converter resolves them
    (KG/convert_weights.py engine_config, KG/PLAN.md:25-44)."""
    from oracle import gemma4 as g4

    L = g4.G4_E2B.layers
    assert len(L) == 35
    assert [l for l, lay in enumerate(L) if not lay.sliding] == [4, 9, 14, 19, 24, 29, 34]
    assert all(lay.kv_layer == l for l, lay in enumerate(L[:15]))
    assert all(lay.kv_layer == (13 if lay.sliding else 14) for lay in L[15:])
    assert {lay.ffn_dim for lay in L[:15]} == {6144} and {lay.ffn_dim for lay in L[15:]} == {12288}
    assert {(lay.head_dim, lay.rope_pairs, lay.rope_theta) for lay in L} == {(256, 128, 1e4), (512, 64, 1e6)}
    invf = g4.G4_E2B.inv_freq(4)
    assert np.count_nonzero(invf) == 64 and invf[63] == np.float32(1e6 ** (-126 / 512))


def test_gemma4_softcap_keeps_the_argmax(rng):
    from oracle import gemma4 as g4

    d = g4.G4Decoder(g4.G4_TINY, g4.make_weights(g4.G4_TINY, 1), 8)
    x = (rng.standard_normal(1000) * 40).astype(np.float32)
    c = d.softcap(x)
    assert np.argmax(c) == np.argmax(x) and np.abs(c).max() < 30
    assert np.allclose(c, 30 * np.tanh(x.astype(np.float64) / 30), rtol=1e-6)
