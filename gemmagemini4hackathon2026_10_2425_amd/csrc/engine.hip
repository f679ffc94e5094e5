// The decode engine: device-resident weights, activations, KV caches and token
// buffer, and the one-token decode step composed from the library's kernels.
//
// Reference: Engine (KL/main.swift:152-347, KG/main.swift:394-457). Step order
// follows encodeDecode (KL/main.swift:321-347) with the Gemma substitutions
// (sqrt(D) embedding scale KG/main.swift:397, GeGLU, tied LM head
// KG/main.swift:379-380, (1 + w) RMSNorm weights), or the Llama ones (plain
// RMSNorm weights, SwiGLU, an untied lm_head KL/main.swift:306, Llama-3 RoPE
// scaling KL/main.swift:96-107). The token of step t is
// written by the GPU into tokens[t + 1] and read from there by step t + 1
// (KL/kernels.metal:343 / :38), so a run of steps needs no host round trip.
//
// MI355X specifics: the engine owns one non-blocking HIP stream (default
// priority). A decode run replays one captured hipGraph per token; inside it
// every kernel reads the step position from a device counter that the final
// argmax advances, so the same graph serves every position.
//
// Prefill (prefill(n:useGemm:), KL/main.swift:357-372, 412-446) runs the
// prompt in chunks of up to prefill_rows() rows through the matrix-core
// products, the causal multi-query attention and row-batched norm / RoPE /
// cast kernels, with the reference's fp16 activation points; the last row of
// the last chunk goes through the decode path's LM head and argmax. The
// ENG_NO_GEMM tunable (the reference's --no-gemm) steps the decode path
// instead.
#include "engine.hpp"

#include <math.h>
#include <stdio.h>
#include <string.h>

using namespace mxd_eng;

namespace {

__global__ void set_int_kernel(int32_t* p, int v) { *p = v; }

// Tensor ids of the synthetic-weight generator: embed 1, final_norm 2,
// lm_head 3 (untied heads only), and 1000 + 16 * layer + {attn_norm 0, wqkv 1,
// wo 2, ffn_norm 3, wgate 4, wup 5, wdown 6}; names follow the reference's
// weight file (KL/convert_weights.py:56-69).
void plan_weights(mxd_engine* e) {
    const mxd_model_config& c = e->c;
    const size_t D = c.dim, F = c.ffn_dim;
    size_t off = 0;
    add_tensor(e, "embed", (size_t)c.vocab * D, MXD_F16, 1, off);
    add_tensor(e, "final_norm", D, MXD_F32, 2, off);
    if (c.untied_lm_head) add_tensor(e, "lm_head", (size_t)c.vocab * D, MXD_F16, 3, off);
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "l" + std::to_string(l) + ".";
        const uint64_t base = 1000 + 16 * (uint64_t)l;
        add_tensor(e, p + "attn_norm", D, MXD_F32, base + 0, off);
        add_tensor(e, p + "wqkv", (size_t)e->qkv_dim() * D, MXD_F16, base + 1, off);
        add_tensor(e, p + "wo", D * (size_t)e->q_dim(), MXD_F16, base + 2, off);
        add_tensor(e, p + "ffn_norm", D, MXD_F32, base + 3, off);
        add_tensor(e, p + "wgate", F * D, MXD_F16, base + 4, off);
        add_tensor(e, p + "wup", F * D, MXD_F16, base + 5, off);
        add_tensor(e, p + "wdown", D * F, MXD_F16, base + 6, off);
    }
    e->wbytes = off;
}

// One decode step: reads tokens[pos], appends K/V at pos, and with `sample`
// writes argmax(logits) to tokens[pos + 1]. With pos_dev the position is read
// on the device and advanced by the argmax (the captured form).
int encode_step(mxd_engine* e, int pos, int32_t* pos_dev, bool sample) {
    if (e->arch == ENG_GEMMA4) return g4_step(e, pos, pos_dev, sample);
    const mxd_model_config& c = e->c;
    hipStream_t s = e->stream;
    mxd_stream_t ms = reinterpret_cast<mxd_stream_t>(s);
    const int D = c.dim, NH = c.n_heads, NKV = c.n_kv_heads, HD = c.head_dim, F = c.ffn_dim, V = c.vocab;
    const float escale = c.embed_scale_sqrt_dim ? sqrtf((float)D) : 1.0f;
    const float ascale = 1.0f / sqrtf((float)HD);
    int rc;
    if ((rc = mxd::embed_dev(e->embed, e->tokens, pos, pos_dev, 1, e->x, D, escale, V, s, e->step))) return rc;
    // Per layer, three launches: [rmsnorm + qkv + rope + append + attention +
    // wo + residual] (attn_block), [rmsnorm + gate_up], [down + residual]; or,
    // unfused, five: [rmsnorm + qkv + rope + append], attention, [wo +
    // residual], [rmsnorm + gate_up], [down + residual].
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerPtrs& Lp = e->L[l];
        if (e->fused) {
            if ((rc = mxd::attn_block(Lp.wqkv, Lp.wo, e->x, Lp.attn_norm, c.rms_eps, c.norm_plus_one, Lp.kc, Lp.vc,
                                      e->invf, NH, NKV, HD, D, e->max_ctx, pos, pos_dev, ascale, e->step, l, e->ab_ws,
                                      e->ab_ws_bytes, s)))
                return rc;
        } else {
            if ((rc = mxd_qkv_rope_kv(Lp.wqkv, e->x, Lp.attn_norm, c.rms_eps, c.norm_plus_one, e->qkv, Lp.kc, Lp.vc,
                                      e->invf, NH, NKV, HD, D, e->max_ctx, pos, pos_dev, ms)))
                return rc;
            if (e->att_splits) {
                // The attention leaves its splits' partials; the o projection
                // merges them as it loads its input (no merge launch).
                float* part = static_cast<float*>(e->attn_ws);
                if ((rc = mxd_attention_split(e->qkv, Lp.kc, Lp.vc, NH, NKV, HD, e->max_ctx, pos + 1, pos_dev, ascale,
                                              e->att_splits, part, e->attn_ws_bytes, ms)))
                    return rc;
                if ((rc = mxd_matvec_f16_attn_merge(Lp.wo, part, e->att_splits, NH, HD, e->max_ctx, pos + 1, pos_dev,
                                                    e->x, D, MXD_EPI_ADD, nullptr, ms)))
                    return rc;
            } else {
                if ((rc = mxd_attention(e->qkv, Lp.kc, Lp.vc, e->att, NH, NKV, HD, e->max_ctx, pos + 1, pos_dev,
                                        ascale, e->attn_ws, e->attn_ws_bytes, ms)))
                    return rc;
                if ((rc = mxd_matvec_f16(Lp.wo, e->att, MXD_F32, e->x, D, e->q_dim(), MXD_EPI_ADD, nullptr, ms)))
                    return rc;
            }
        }
        if ((rc = mxd_gate_up_rmsnorm(Lp.wgate, Lp.wup, e->x, Lp.ffn_norm, c.rms_eps, c.norm_plus_one, e->h, F, D,
                                      c.act, ms)))
            return rc;
        if ((rc = mxd_matvec_f16(Lp.wdown, e->h, MXD_F32, e->x, D, F, MXD_EPI_ADD, nullptr, ms))) return rc;
    }
    if (!sample) return MXD_OK;
    if ((rc = mxd_matvec_f16_rmsnorm(e->head, e->x, e->final_norm, c.rms_eps, c.norm_plus_one, e->logits, V, D,
                                     MXD_EPI_STORE, nullptr, ms)))
        return rc;
    return mxd::argmax_dev(e->logits, e->tokens, V, pos + 1, pos_dev, pos_dev != nullptr, e->am_ws, s,
                           pos_dev ? e->htokens_dev : nullptr);
}

// The batched prefill of tokens[pos0 .. pos0 + T) (encodePrefillChunk,
// KL/main.swift:412-446); with sample, tokens[pos0 + T] = argmax of the last
// row's logits, which stay in e->logits.
int encode_prefill(mxd_engine* e, int pos0, int T, bool sample) {
    const mxd_model_config& c = e->c;
    hipStream_t s = e->stream;
    mxd_stream_t ms = reinterpret_cast<mxd_stream_t>(s);
    const int D = c.dim, NH = c.n_heads, NKV = c.n_kv_heads, HD = c.head_dim, F = c.ffn_dim, V = c.vocab;
    const int QKV = e->qkv_dim(), QD = e->q_dim();
    const float escale = c.embed_scale_sqrt_dim ? sqrtf((float)D) : 1.0f;
    const float ascale = 1.0f / sqrtf((float)HD);
    void* ws = e->gm_ws;
    const size_t wsb = e->gm_ws_bytes;
    int rc;
    if ((rc = mxd::embed_dev(e->embed, e->tokens, pos0, nullptr, T, e->bx, D, escale, V, s))) return rc;
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerPtrs& Lp = e->L[l];
        if ((rc = mxd_rmsnorm(e->bx, Lp.attn_norm, e->bxn, MXD_F16, T, D, c.rms_eps, c.norm_plus_one, ms))) return rc;
        if ((rc = mxd_gemm_f16(Lp.wqkv, e->bxn, MXD_F16, e->bqkv, T, QKV, D, MXD_EPI_STORE, ws, wsb, ms))) return rc;
        if ((rc = mxd_rope_kv(e->bqkv, Lp.kc, Lp.vc, e->invf, NH, NKV, HD, e->max_ctx, pos0, T, ms))) return rc;
        // The attention rows and the hidden rows are rounded to fp16 where
        // they are written (the reference's attHalf / hidHalf casts), in the
        // fp32 buffers' memory, so the o and down products stage fp16 rows.
        uint16_t* batt_h = reinterpret_cast<uint16_t*>(e->batt);
        if ((rc = mxd::attention_prefill_h16(e->bqkv, QKV, Lp.kc, Lp.vc, batt_h, QD, NH, NKV, HD, e->max_ctx, pos0, T,
                                             0, ascale, s)))
            return rc;
        if ((rc = mxd_gemm_f16(Lp.wo, batt_h, MXD_F16, e->bx, T, D, QD, MXD_EPI_ADD, ws, wsb, ms))) return rc;
        if ((rc = mxd_rmsnorm(e->bx, Lp.ffn_norm, e->bxn, MXD_F16, T, D, c.rms_eps, c.norm_plus_one, ms))) return rc;
        if (mxd::gemm_on_matrix_cores(T, D)) {
            uint16_t* bh_h = reinterpret_cast<uint16_t*>(e->bh);
            if ((rc = mxd::gemm_gate_up_f16_h16(Lp.wgate, Lp.wup, e->bxn, bh_h, T, F, D, c.act, ws, wsb, s))) return rc;
            if ((rc = mxd_gemm_f16(Lp.wdown, bh_h, MXD_F16, e->bx, T, D, F, MXD_EPI_ADD, ws, wsb, ms))) return rc;
        } else {  // per-row matvecs: fp32 hidden rows, rounded as the down product loads them
            if ((rc = mxd_gemm_gate_up_f16(Lp.wgate, Lp.wup, e->bxn, e->bh, T, F, D, c.act, ws, wsb, ms))) return rc;
            if ((rc = mxd_gemm_f16(Lp.wdown, e->bh, MXD_F32, e->bx, T, D, F, MXD_EPI_ADD, ws, wsb, ms))) return rc;
        }
    }
    if (!sample) return MXD_OK;
    // Only the last row needs logits: it takes the decode path's head.
    HIP_OK(hipMemcpyAsync(e->x, e->bx + (size_t)(T - 1) * D, (size_t)D * 4, hipMemcpyDeviceToDevice, s),
           "mxd_engine_prefill");
    if ((rc = mxd_matvec_f16_rmsnorm(e->head, e->x, e->final_norm, c.rms_eps, c.norm_plus_one, e->logits, V, D,
                                     MXD_EPI_STORE, nullptr, ms)))
        return rc;
    return mxd::argmax_dev(e->logits, e->tokens, V, pos0 + T, nullptr, false, e->am_ws, s);
}

// Split-K workspace the prefill products may need for any chunk of 1 .. rows rows.
size_t prefill_ws_bytes(const mxd_model_config& c, int qkv_dim, int q_dim, int rows) {
    size_t m = 0;
    for (int T = 1; T <= rows; ++T) {
        m = max(m, mxd_gemm_f16_workspace_size(T, qkv_dim, c.dim));
        m = max(m, mxd_gemm_f16_workspace_size(T, c.dim, q_dim));
        m = max(m, mxd_gemm_gate_up_f16_workspace_size(T, c.ffn_dim, c.dim));
        m = max(m, mxd_gemm_f16_workspace_size(T, c.dim, c.ffn_dim));
    }
    return m;
}

// theta^(-2i/hd), and under Llama-3 scaling: kept when its wavelength 2 pi / f
// is below original / high_freq_factor, divided by factor above
// original / low_freq_factor, and blended linearly in original / wavelength in
// between.
double rope_inv_freq(const mxd_model_config& c, int i) {
    const double f = 1.0 / pow((double)c.rope_theta, (double)(2 * i) / (double)c.head_dim);
    if (c.rope_factor <= 0.0f) return f;
    const double orig = (double)c.rope_original_max_positions, factor = (double)c.rope_factor;
    const double lo = (double)c.rope_low_freq_factor, hi = (double)c.rope_high_freq_factor;
    const double wave = 2.0 * M_PI / f;
    if (wave < orig / hi) return f;
    if (wave > orig / lo) return f / factor;
    const double t = (orig / wave - lo) / (hi - lo);
    return (1.0 - t) * f / factor + t * f;
}

int check_config(const mxd_model_config* c, int max_ctx) {
    MXD_REQUIRE(c, MXD_ERR_INVALID_ARG, "mxd_engine_create: null config");
    MXD_REQUIRE(c->n_layers > 0 && c->dim > 0 && c->n_heads > 0 && c->n_kv_heads > 0 && c->head_dim > 0 &&
                    c->ffn_dim > 0 && c->vocab > 0,
                MXD_ERR_INVALID_ARG, "mxd_engine_create: sizes must be positive");
    MXD_REQUIRE(c->n_heads % c->n_kv_heads == 0, MXD_ERR_INVALID_ARG, "mxd_engine_create: n_heads %% n_kv_heads != 0");
    MXD_REQUIRE(c->head_dim == 64 || c->head_dim == 128 || c->head_dim == 256, MXD_ERR_UNSUPPORTED,
                "mxd_engine_create: head_dim %d (64, 128 or 256)", c->head_dim);
    MXD_REQUIRE(c->rope_factor <= 0.0f ||
                    (c->rope_factor >= 1.0f && c->rope_low_freq_factor > 0.0f &&
                     c->rope_high_freq_factor > c->rope_low_freq_factor && c->rope_original_max_positions > 0),
                MXD_ERR_INVALID_ARG,
                "mxd_engine_create: llama3 rope scaling needs factor >= 1, 0 < low_freq_factor < high_freq_factor "
                "and original_max_positions > 0");
    MXD_REQUIRE(c->dim % 8 == 0 && c->ffn_dim % 8 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_engine_create: dim and ffn_dim must be multiples of 8");
    MXD_REQUIRE(c->act == MXD_ACT_GELU_TANH || c->act == MXD_ACT_SILU, MXD_ERR_INVALID_ARG,
                "mxd_engine_create: act %d", c->act);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_engine_create: max_ctx=%d must be a positive multiple of 32", max_ctx);
    return MXD_OK;
}

}  // namespace

int mxd_eng::allocate(mxd_engine* e) {
    hipError_t he;
    if ((he = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking)) != hipSuccess ||
        (he = hipMalloc(&e->wbase, e->wbytes)) != hipSuccess || (he = hipMalloc(&e->abase, e->abytes)) != hipSuccess ||
        (he = hipHostMalloc(reinterpret_cast<void**>(&e->htokens), ((size_t)e->max_ctx + 1) * 4,
                            hipHostMallocMapped | hipHostMallocCoherent)) != hipSuccess ||
        (he = hipHostGetDevicePointer(reinterpret_cast<void**>(&e->htokens_dev), e->htokens, 0)) != hipSuccess) {
        const size_t wb = e->wbytes, ab = e->abytes;
        destroy(e);
        return mxd::fail(MXD_ERR_ALLOC, "mxd_engine_create: %s (weights %zu B, buffers %zu B)", hipGetErrorString(he),
                         wb, ab);
    }
    for (hipEvent_t& ev : e->step_done) {
        if ((he = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) {
            destroy(e);
            return mxd::fail(MXD_ERR_HIP, "mxd_engine_create: %s", hipGetErrorString(he));
        }
    }
    // Zero every buffer once (caches, token buffer, argmax workspace), off any graph.
    if ((he = hipMemsetAsync(e->abase, 0, e->abytes, e->stream)) != hipSuccess) {
        destroy(e);
        return mxd::fail(MXD_ERR_HIP, "mxd_engine_create: %s", hipGetErrorString(he));
    }
    return MXD_OK;
}

extern "C" int mxd_engine_create(const mxd_model_config* cfg, int max_ctx, mxd_engine** out) {
    MXD_REQUIRE(out, MXD_ERR_INVALID_ARG, "mxd_engine_create: null out");
    *out = nullptr;
    if (int rc = check_config(cfg, max_ctx)) return rc;
    mxd_engine* e = new mxd_engine();
    e->c = *cfg;
    e->max_ctx = max_ctx;
    const mxd_model_config& c = e->c;
    plan_weights(e);

    // Activations, caches and small buffers share one allocation.
    const size_t D = c.dim, F = c.ffn_dim;
    const size_t kv_bytes = (size_t)c.n_kv_heads * max_ctx * c.head_dim * 2;
    e->attn_ws_bytes = mxd_attention_workspace_size(c.n_heads, c.n_kv_heads, c.head_dim, max_ctx);
    {
        // One 32-key block per wave (4 waves per split) over the whole
        // context; folded into the o projection while that is at most 8
        // splits (contexts of up to 1024 keys) and more than one. A folded
        // attention takes at least ENG_ATT_SPLITS (default 6) splits: spread
        // over more workgroups, the same blocks finish sooner (Gemma-2B at
        // max_ctx 384, measured on MI355X: 858-859 tok/s with 6 or 8 splits
        // against 849-850 with the 3 one block per wave needs).
        // ENG_ATT_FOLD = 3 also folds longer contexts, as 8 splits (at
        // max_ctx 4096: 861 against 814 tok/s at 129-384 keys, but 760
        // against 816 at 3584-3840 keys, where each wave walks ~4 blocks).
        int splits = ((max_ctx + 31) / 32 + 3) / 4;
        if (mxd::tunable("ENG_ATT_FOLD", 1) == 3 && splits > 8) splits = 8;
        if (splits >= 2 && splits <= 8) splits = max(splits, min(8, mxd::tunable("ENG_ATT_SPLITS", 6)));
        e->att_splits = splits >= 2 && splits <= 8 && mxd::tunable("ENG_ATT_FOLD", 1) != 2 ? splits : 0;
        const size_t need = (size_t)splits * c.n_heads * (c.head_dim + 2) * sizeof(float);
        if (e->att_splits && e->attn_ws_bytes < need) e->attn_ws_bytes = need;
    }
    // The fused attention block (ENG_FUSED = 1) takes the attention half of
    // every layer in one launch (models of at most 64 layers and attention
    // heads of at most 8192 values). Off by default: measured on MI355X, its
    // in-kernel handoffs between XCDs cost more than the kernel boundaries
    // they replace (Gemma-2B layer: 31 us against 18.8 us for the three
    // launches; per-workgroup stamps put 5-12 us on each handoff).
    e->fused = mxd::tunable("ENG_FUSED", 2) == 1 && c.n_layers <= 64 && c.n_heads * c.head_dim <= 8192;
    e->ab_ws_bytes = e->fused ? mxd::attn_block_workspace_size(c.n_heads, c.n_kv_heads, c.head_dim, max_ctx) : 0;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t o_x = take(D * 4), o_xn = take(D * 4), o_qkv = take((size_t)e->qkv_dim() * 4);
    const size_t o_att = take((size_t)e->q_dim() * 4), o_h = take(F * 4), o_logits = take((size_t)c.vocab * 4);
    const size_t o_invf = take((size_t)c.head_dim / 2 * 4), o_tok = take(((size_t)max_ctx + 1) * 4), o_pos = take(4);
    const size_t o_aws = take(e->attn_ws_bytes), o_am = take(mxd_argmax_workspace_size(c.vocab));
    const size_t o_abws = take(max(e->ab_ws_bytes, (size_t)16)), o_step = take(4);
    const size_t B = (size_t)(e->max_rows = min(prefill_rows(), max_ctx));
    e->gm_ws_bytes = prefill_ws_bytes(c, e->qkv_dim(), e->q_dim(), e->max_rows);
    const size_t o_bx = take(B * D * 4), o_bxn = take(B * D * 2), o_bqkv = take(B * e->qkv_dim() * 4);
    const size_t o_batt = take(B * e->q_dim() * 4);
    const size_t o_bh = take(B * F * 4), o_gws = take(max(e->gm_ws_bytes, (size_t)16));
    std::vector<size_t> o_kc(c.n_layers), o_vc(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        o_kc[l] = take(kv_bytes);
        o_vc[l] = take(kv_bytes);
    }
    e->abytes = off;

    if (int rc = allocate(e)) return rc;
    char* a = e->abase;
    e->x = reinterpret_cast<float*>(a + o_x);
    e->xn = reinterpret_cast<float*>(a + o_xn);
    e->qkv = reinterpret_cast<float*>(a + o_qkv);
    e->att = reinterpret_cast<float*>(a + o_att);
    e->h = reinterpret_cast<float*>(a + o_h);
    e->logits = reinterpret_cast<float*>(a + o_logits);
    e->invf = reinterpret_cast<float*>(a + o_invf);
    e->tokens = reinterpret_cast<int32_t*>(a + o_tok);
    e->pos = reinterpret_cast<int32_t*>(a + o_pos);
    e->attn_ws = a + o_aws;
    e->am_ws = a + o_am;
    e->step = reinterpret_cast<int32_t*>(a + o_step);
    if (e->fused) {
        e->ab_ws = a + o_abws;
        e->ab_err = mxd::attn_block_err(e->ab_ws, c.n_heads, c.n_kv_heads, c.head_dim, max_ctx);
    }
    e->bx = reinterpret_cast<float*>(a + o_bx);
    e->bxn = reinterpret_cast<uint16_t*>(a + o_bxn);
    e->bqkv = reinterpret_cast<float*>(a + o_bqkv);
    e->batt = reinterpret_cast<float*>(a + o_batt);
    e->bh = reinterpret_cast<float*>(a + o_bh);
    e->gm_ws = a + o_gws;
    e->embed = wptr<uint16_t>(e, "embed");
    e->head = c.untied_lm_head ? wptr<uint16_t>(e, "lm_head") : e->embed;
    e->final_norm = wptr<float>(e, "final_norm");
    e->L.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "l" + std::to_string(l) + ".";
        LayerPtrs& Lp = e->L[l];
        Lp.attn_norm = wptr<float>(e, p + "attn_norm");
        Lp.ffn_norm = wptr<float>(e, p + "ffn_norm");
        Lp.wqkv = wptr<uint16_t>(e, p + "wqkv");
        Lp.wo = wptr<uint16_t>(e, p + "wo");
        Lp.wgate = wptr<uint16_t>(e, p + "wgate");
        Lp.wup = wptr<uint16_t>(e, p + "wup");
        Lp.wdown = wptr<uint16_t>(e, p + "wdown");
        Lp.kc = reinterpret_cast<uint16_t*>(a + o_kc[l]);
        Lp.vc = reinterpret_cast<uint16_t*>(a + o_vc[l]);
    }
    // RoPE inverse frequencies in double, stored as float (KL/main.swift:92-94),
    // with the Llama-3 band scaling when configured (KL/main.swift:96-107).
    std::vector<float> invf(c.head_dim / 2);
    for (int i = 0; i < c.head_dim / 2; ++i) invf[i] = (float)rope_inv_freq(c, i);
    hipError_t he = hipMemcpyAsync(e->invf, invf.data(), invf.size() * 4, hipMemcpyHostToDevice, e->stream);
    if (he == hipSuccess) he = hipStreamSynchronize(e->stream);
    if (he != hipSuccess) {
        destroy(e);
        return mxd::fail(MXD_ERR_HIP, "mxd_engine_create: %s", hipGetErrorString(he));
    }
    *out = e;
    return MXD_OK;
}

extern "C" int mxd_engine_destroy(mxd_engine* e) {
    if (e) {
        (void)hipStreamSynchronize(e->stream);
        destroy(e);
    }
    return MXD_OK;
}

extern "C" int mxd_engine_num_tensors(const mxd_engine* e) { return e ? (int)e->tensors.size() : 0; }

extern "C" int mxd_engine_tensor(const mxd_engine* e, int i, const char** name, void** dev_ptr, size_t* bytes,
                                 int* dtype) {
    MXD_REQUIRE(e && i >= 0 && i < (int)e->tensors.size(), MXD_ERR_INVALID_ARG, "mxd_engine_tensor: index %d", i);
    const TensorInfo& t = e->tensors[i];
    if (name) *name = t.name.c_str();
    if (dev_ptr) *dev_ptr = e->wbase + t.offset;
    if (bytes) *bytes = t.bytes;
    if (dtype) *dtype = t.dtype;
    return MXD_OK;
}

extern "C" int mxd_engine_find_tensor(const mxd_engine* e, const char* name) {
    if (!e || !name) return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_engine_find_tensor: null argument");
    auto it = e->index.find(name);
    if (it == e->index.end()) return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_engine_find_tensor: no tensor %s", name);
    return it->second;
}

extern "C" int mxd_engine_init_random(mxd_engine* e, uint64_t seed, float stddev) {
    MXD_REQUIRE(e, MXD_ERR_INVALID_ARG, "mxd_engine_init_random: null engine");
    for (const TensorInfo& t : e->tensors) {
        const uint64_t n = t.bytes / (t.dtype == MXD_F32 ? 4 : 2);
        if (int rc = mxd::fill_normal_dev(e->wbase + t.offset, t.dtype, n, seed, t.id, stddev, t.shift, e->stream))
            return rc;
    }
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_init_random");
    return MXD_OK;
}

extern "C" int mxd_engine_fill_tensor(mxd_engine* e, int i, uint64_t seed, float stddev) {
    MXD_REQUIRE(e && i >= 0 && i < (int)e->tensors.size(), MXD_ERR_INVALID_ARG, "mxd_engine_fill_tensor: index %d",
                i);
    const TensorInfo& t = e->tensors[i];
    const uint64_t n = t.bytes / (t.dtype == MXD_F32 ? 4 : 2);
    if (int rc = mxd::fill_normal_dev(e->wbase + t.offset, t.dtype, n, seed, t.id, stddev, t.shift, e->stream))
        return rc;
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_fill_tensor");
    return MXD_OK;
}

extern "C" int mxd_engine_upload(mxd_engine* e, int i, const void* host, size_t bytes) {
    MXD_REQUIRE(e && host && i >= 0 && i < (int)e->tensors.size(), MXD_ERR_INVALID_ARG,
                "mxd_engine_upload: bad arguments");
    MXD_REQUIRE(bytes == e->tensors[i].bytes, MXD_ERR_INVALID_ARG, "mxd_engine_upload: %s has %zu bytes, got %zu",
                e->tensors[i].name.c_str(), e->tensors[i].bytes, bytes);
    HIP_OK(hipMemcpyAsync(e->wbase + e->tensors[i].offset, host, bytes, hipMemcpyHostToDevice, e->stream),
           "mxd_engine_upload");
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_upload");
    return MXD_OK;
}

extern "C" int mxd_engine_download(mxd_engine* e, int i, void* host, size_t bytes) {
    MXD_REQUIRE(e && host && i >= 0 && i < (int)e->tensors.size(), MXD_ERR_INVALID_ARG,
                "mxd_engine_download: bad arguments");
    MXD_REQUIRE(bytes == e->tensors[i].bytes, MXD_ERR_INVALID_ARG, "mxd_engine_download: %s has %zu bytes, got %zu",
                e->tensors[i].name.c_str(), e->tensors[i].bytes, bytes);
    HIP_OK(hipMemcpyAsync(host, e->wbase + e->tensors[i].offset, bytes, hipMemcpyDeviceToHost, e->stream),
           "mxd_engine_download");
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_download");
    return MXD_OK;
}

extern "C" int mxd_engine_set_tokens(mxd_engine* e, const int32_t* ids, int start, int n) {
    MXD_REQUIRE(e && ids && start >= 0 && n >= 0 && start + n <= e->max_ctx + 1, MXD_ERR_INVALID_ARG,
                "mxd_engine_set_tokens: range [%d, %d) outside [0, %d]", start, start + n, e ? e->max_ctx + 1 : 0);
    for (int i = 0; i < n; ++i)
        MXD_REQUIRE(ids[i] >= 0 && ids[i] < e->c.vocab, MXD_ERR_INVALID_ARG,
                    "mxd_engine_set_tokens: token id %d out of range", ids[i]);
    HIP_OK(hipMemcpyAsync(e->tokens + start, ids, (size_t)n * 4, hipMemcpyHostToDevice, e->stream),
           "mxd_engine_set_tokens");
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_set_tokens");
    return MXD_OK;
}

extern "C" int mxd_engine_get_tokens(mxd_engine* e, int32_t* ids, int start, int n) {
    MXD_REQUIRE(e && ids && start >= 0 && n >= 0 && start + n <= e->max_ctx + 1, MXD_ERR_INVALID_ARG,
                "mxd_engine_get_tokens: bad range");
    HIP_OK(hipMemcpyAsync(ids, e->tokens + start, (size_t)n * 4, hipMemcpyDeviceToHost, e->stream),
           "mxd_engine_get_tokens");
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_get_tokens");
    return MXD_OK;
}

extern "C" int mxd_engine_get_logits(mxd_engine* e, float* host) {
    MXD_REQUIRE(e && host, MXD_ERR_INVALID_ARG, "mxd_engine_get_logits: null argument");
    HIP_OK(hipMemcpyAsync(host, e->logits, (size_t)e->c.vocab * 4, hipMemcpyDeviceToHost, e->stream),
           "mxd_engine_get_logits");
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_get_logits");
    // Gemma-4's final softcap, applied to the dumped logits on the host as the
    // reference's --dump-logits does (KG/main.swift:657-662); argmax ran on
    // the raw logits (the cap is monotonic).
    const float cap = e->arch == ENG_GEMMA4 ? e->g4.softcap : 0.0f;
    if (cap > 0.0f)
        for (int i = 0; i < e->c.vocab; ++i) host[i] = cap * tanhf(host[i] / cap);
    return MXD_OK;
}

extern "C" int mxd_engine_step(mxd_engine* e, int pos, int sample) {
    MXD_REQUIRE(e, MXD_ERR_INVALID_ARG, "mxd_engine_step: null engine");
    MXD_REQUIRE(pos >= 0 && pos < e->max_ctx, MXD_ERR_INVALID_ARG, "mxd_engine_step: pos %d outside [0, %d)", pos,
                e->max_ctx);
    return encode_step(e, pos, nullptr, sample != 0);
}

extern "C" int mxd_engine_prefill(mxd_engine* e, int n) {
    MXD_REQUIRE(e && n >= 1 && n <= e->max_ctx, MXD_ERR_INVALID_ARG, "mxd_engine_prefill: n=%d", n);
    if (e->arch == ENG_GEMMA4) return g4_prefill(e, n);
    if (n > 1 && mxd::tunable("ENG_NO_GEMM", 0) != 1) {
        for (int done = 0; done < n;) {
            const int rows = min(e->max_rows, n - done);
            if (int rc = encode_prefill(e, done, rows, done + rows == n)) return rc;
            done += rows;
        }
        return MXD_OK;
    }
    for (int p = 0; p < n; ++p)
        if (int rc = encode_step(e, p, nullptr, p == n - 1)) return rc;
    return MXD_OK;
}

extern "C" int mxd_engine_decode(mxd_engine* e, int pos, int count) {
    MXD_REQUIRE(e, MXD_ERR_INVALID_ARG, "mxd_engine_decode: null engine");
    MXD_REQUIRE(pos >= 0 && count >= 0 && pos + count <= e->max_ctx, MXD_ERR_INVALID_ARG,
                "mxd_engine_decode: steps %d..%d exceed max_ctx %d", pos, pos + count - 1, e->max_ctx);
    if (count == 0) return MXD_OK;
    if (!e->graph) {
        hipGraph_t g = nullptr;
        HIP_OK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "mxd_engine_decode: begin capture");
        const int rc = encode_step(e, 0, e->pos, true);
        const hipError_t ce = hipStreamEndCapture(e->stream, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        HIP_OK(ce, "mxd_engine_decode: end capture");
        const hipError_t ie = hipGraphInstantiate(&e->graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        HIP_OK(ie, "mxd_engine_decode: instantiate");
    }
    if (pos != e->pos_next) {
        hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, e->stream, e->pos, pos);
        if (int rc = mxd::check_launch("mxd_engine_decode")) return rc;
    }
    e->pos_next = -1;  // until every launch below went out
    for (int i = 0; i < count; ++i) {
        HIP_OK(hipGraphLaunch(e->graph, e->stream), "mxd_engine_decode: graph launch");
        HIP_OK(hipEventRecord(e->step_done[(pos + i) % mxd_engine::RING], e->stream), "mxd_engine_decode: event");
    }
    e->pos_next = pos + count;
    return MXD_OK;
}

extern "C" int mxd_engine_wait_token(mxd_engine* e, int pos, int32_t* token) {
    MXD_REQUIRE(e && token, MXD_ERR_INVALID_ARG, "mxd_engine_wait_token: null argument");
    MXD_REQUIRE(pos >= 0 && pos < e->max_ctx, MXD_ERR_INVALID_ARG, "mxd_engine_wait_token: pos %d outside [0, %d)",
                pos, e->max_ctx);
    // The ring slot of pos holds its step's event, or that of a later step
    // queued since (then the wait is longer, never too short: one stream).
    HIP_OK(hipEventSynchronize(e->step_done[pos % mxd_engine::RING]), "mxd_engine_wait_token");
    *token = __atomic_load_n(&e->htokens[pos + 1], __ATOMIC_ACQUIRE);
    return MXD_OK;
}

extern "C" int mxd_engine_sync(mxd_engine* e) {
    MXD_REQUIRE(e, MXD_ERR_INVALID_ARG, "mxd_engine_sync: null engine");
    HIP_OK(hipStreamSynchronize(e->stream), "mxd_engine_sync");
    if (e->ab_err) {
        int err = 0;
        HIP_OK(hipMemcpy(&err, e->ab_err, sizeof(int), hipMemcpyDeviceToHost), "mxd_engine_sync");
        MXD_REQUIRE(err == 0, MXD_ERR_HIP, "mxd_engine_sync: a wait between workgroups of the fused attention block "
                                           "ran out (results of this run are not valid)");
    }
    return MXD_OK;
}

extern "C" size_t mxd_engine_weight_bytes(const mxd_engine* e) { return e ? e->wbytes : 0; }
