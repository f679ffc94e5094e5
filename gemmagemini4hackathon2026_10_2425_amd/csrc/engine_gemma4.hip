// The Gemma-4 decode engine behind the mxd_engine handle.
//
// Reference: the Gemma-4 E2B engine (KG = ios_kernels/kernels/
// google__gemma-4-E2B-it/kernel_metal_f16_20261025-1225/): Engine
// (KG/main.swift:148-457), the decode order of encodeDecode
// (KG/main.swift:394-423) and the per-layer facts of the weight file's
// "engine" header (KG/main.swift:75-101, KG/convert_weights.py engine_config).
// Per layer, in order:
//   [q|k|v] = Wqkv . rmsnorm(x, attn_norm)          (matvec with fused norm)
//   per-head q/k/v norm, RoPE on rope_pairs pairs,  (mxd_qk_norm_rope_kv)
//     k, v appended (own cache only)
//   att = attention(q, cache of kv_layer), scale 1, (mxd_attention_window)
//     the last `window` keys on sliding layers
//   x += rmsnorm(Wo . att, post_attn_norm)          (matvec, mxd_rmsnorm_add)
//   h = gelu(Wg . xn) * (Wu . xn), xn = rmsnorm(x, ffn_norm)
//   x += rmsnorm(Wdown . h, post_ffn_norm)
//   g = gelu(Wple_gate . x) * ple[l]                (matvec, GELU_MUL epilogue)
//   x = (x + rmsnorm(Wple_out . g, post_ple_norm)) * layer_scalar
// with the per-layer inputs ple = (rmsnorm(Wple_proj . x0 / sqrt(D)) *
// ple_norm + ple_embed[tok] * sqrt(P)) / sqrt(2) computed once per token, and
// the tied LM head + argmax after the final norm. Every launch reads the
// position from the device counter under graph capture, as the Llama /
// Gemma step does (engine.hip).
#include "engine.hpp"

#include <math.h>
#include <string.h>

#include <utility>

using namespace mxd_eng;

namespace {

constexpr int G4_FREQS = 256;  // inverse-frequency slots per layer (head_dim up to 512)

bool owns_kv(const mxd_engine* e, int l) { return e->g4l[l].kv_layer == l; }
int g4_q_dim(const mxd_engine* e, int l) { return e->g4.n_heads * e->g4l[l].head_dim; }
int g4_qkv_dim(const mxd_engine* e, int l) {
    return (e->g4.n_heads + (owns_kv(e, l) ? 2 * e->g4.n_kv_heads : 0)) * e->g4l[l].head_dim;
}

int g4_check(const mxd_gemma4_config* c, int max_ctx) {
    MXD_REQUIRE(c && c->layers, MXD_ERR_INVALID_ARG, "mxd_engine_create_gemma4: null config or layers");
    MXD_REQUIRE(c->n_layers > 0 && c->dim > 0 && c->n_heads > 0 && c->n_kv_heads > 0 && c->vocab > 0 &&
                    c->ple_dim > 0 && c->ple_vocab > 0 && c->window >= 0,
                MXD_ERR_INVALID_ARG, "mxd_engine_create_gemma4: sizes must be positive");
    MXD_REQUIRE(c->n_heads % c->n_kv_heads == 0, MXD_ERR_INVALID_ARG,
                "mxd_engine_create_gemma4: n_heads %% n_kv_heads != 0");
    const int G = c->n_heads / c->n_kv_heads;
    MXD_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, MXD_ERR_UNSUPPORTED,
                "mxd_engine_create_gemma4: group size %d (1, 2, 4 or 8)", G);
    MXD_REQUIRE(c->dim % 8 == 0 && c->ple_dim % 8 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_engine_create_gemma4: dim and ple_dim must be multiples of 8");
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_engine_create_gemma4: max_ctx=%d must be a positive multiple of 32", max_ctx);
    for (int l = 0; l < c->n_layers; ++l) {
        const mxd_gemma4_layer& y = c->layers[l];
        MXD_REQUIRE(y.head_dim == 64 || y.head_dim == 128 || y.head_dim == 256 || y.head_dim == 512,
                    MXD_ERR_UNSUPPORTED, "mxd_engine_create_gemma4: layer %d head_dim %d (64, 128, 256 or 512)", l,
                    y.head_dim);
        MXD_REQUIRE(y.ffn_dim > 0 && y.ffn_dim % 8 == 0, MXD_ERR_UNSUPPORTED,
                    "mxd_engine_create_gemma4: layer %d ffn_dim %d (a positive multiple of 8)", l, y.ffn_dim);
        MXD_REQUIRE(y.kv_layer >= 0 && y.kv_layer <= l, MXD_ERR_INVALID_ARG,
                    "mxd_engine_create_gemma4: layer %d kv_layer %d (an earlier layer or itself)", l, y.kv_layer);
        const mxd_gemma4_layer& o = c->layers[y.kv_layer];
        MXD_REQUIRE(o.kv_layer == y.kv_layer && o.head_dim == y.head_dim, MXD_ERR_INVALID_ARG,
                    "mxd_engine_create_gemma4: layer %d reads layer %d's cache, which it must own with the same "
                    "head_dim",
                    l, y.kv_layer);
        MXD_REQUIRE(y.rope_pairs >= 0 && y.rope_pairs <= y.head_dim / 2 && (y.rope_pairs == 0 || y.rope_theta > 0.0f),
                    MXD_ERR_INVALID_ARG, "mxd_engine_create_gemma4: layer %d rope_pairs %d / rope_theta %g", l,
                    y.rope_pairs, (double)y.rope_theta);
    }
    return MXD_OK;
}

// Tensor names and shapes of the reference's converted file
// (KG/convert_weights.py); ids of the synthetic-weight generator: embed 1,
// final_norm 2, ple_embed 4, ple_proj 5, ple_norm 6, layer l: 1000 + 16 l +
// {attn_norm 0, wqkv 1, wo 2, ffn_norm 3, wgate 4, wup 5, wdown 6, q_norm 7,
// k_norm 8, post_attn_norm 9, post_ffn_norm 10, ple_gate 11, ple_out 12,
// post_ple_norm 13}. Norm weights multiply unshifted, so their synthetic
// values are 1 + N(0, s^2).
void g4_plan(mxd_engine* e) {
    const mxd_gemma4_config& c = e->g4;
    const size_t D = c.dim, P = c.ple_dim, LP = (size_t)c.n_layers * c.ple_dim;
    size_t off = 0;
    add_tensor(e, "embed", (size_t)c.vocab * D, MXD_F16, 1, off);
    add_tensor(e, "ple_embed", (size_t)c.ple_vocab * LP, MXD_F16, 4, off);
    add_tensor(e, "ple_proj", LP * D, MXD_F16, 5, off);
    add_tensor(e, "ple_norm", P, MXD_F32, 6, off, 1.0f);
    for (int l = 0; l < c.n_layers; ++l) {
        const mxd_gemma4_layer& y = e->g4l[l];
        const std::string p = "l" + std::to_string(l) + ".";
        const uint64_t base = 1000 + 16 * (uint64_t)l;
        const size_t hd = y.head_dim, F = y.ffn_dim;
        add_tensor(e, p + "attn_norm", D, MXD_F32, base + 0, off, 1.0f);
        add_tensor(e, p + "wqkv", (size_t)g4_qkv_dim(e, l) * D, MXD_F16, base + 1, off);
        add_tensor(e, p + "q_norm", hd, MXD_F32, base + 7, off, 1.0f);
        if (owns_kv(e, l)) add_tensor(e, p + "k_norm", hd, MXD_F32, base + 8, off, 1.0f);
        add_tensor(e, p + "wo", D * (size_t)g4_q_dim(e, l), MXD_F16, base + 2, off);
        add_tensor(e, p + "post_attn_norm", D, MXD_F32, base + 9, off, 1.0f);
        add_tensor(e, p + "ffn_norm", D, MXD_F32, base + 3, off, 1.0f);
        add_tensor(e, p + "wgate", F * D, MXD_F16, base + 4, off);
        add_tensor(e, p + "wup", F * D, MXD_F16, base + 5, off);
        add_tensor(e, p + "wdown", D * F, MXD_F16, base + 6, off);
        add_tensor(e, p + "post_ffn_norm", D, MXD_F32, base + 10, off, 1.0f);
        add_tensor(e, p + "ple_gate", P * D, MXD_F16, base + 11, off);
        add_tensor(e, p + "ple_out", D * P, MXD_F16, base + 12, off);
        add_tensor(e, p + "post_ple_norm", D, MXD_F32, base + 13, off, 1.0f);
    }
    add_tensor(e, "final_norm", D, MXD_F32, 2, off, 1.0f);
    e->wbytes = off;
}

}  // namespace

int mxd_eng::g4_step(mxd_engine* e, int pos, int32_t* pos_dev, bool sample) {
    const mxd_gemma4_config& c = e->g4;
    hipStream_t s = e->stream;
    mxd_stream_t ms = reinterpret_cast<mxd_stream_t>(s);
    const int D = c.dim, NH = c.n_heads, NKV = c.n_kv_heads, P = c.ple_dim, L = c.n_layers, V = c.vocab;
    const float eps = c.rms_eps;
    int rc;
    // x = E[tok] * sqrt(D); the per-layer inputs of the token (KG/main.swift:396-399)
    if ((rc = mxd::embed_dev(e->embed, e->tokens, pos, pos_dev, 1, e->x, D, sqrtf((float)D), V, s, e->step)))
        return rc;
    if ((rc = mxd::embed_dev(e->ple_embed, e->tokens, pos, pos_dev, 1, e->ple, L * P, sqrtf((float)P), c.ple_vocab,
                             s)))
        return rc;
    if ((rc = mxd_matvec_f16(e->ple_proj, e->x, MXD_F32, e->pleproj, L * P, D, MXD_EPI_STORE, nullptr, ms))) return rc;
    if ((rc = mxd_ple_combine(e->pleproj, e->ple, e->ple_norm, 1, L, P, 1.0f / sqrtf((float)D), eps, ms))) return rc;
    // Each sandwich norm's residual add, x = (x + rmsnorm(tmp) * w) * post, is
    // folded into the product that reads x next (the *_residual entry
    // points); the updated residual goes to the other of two buffers, since
    // the product's other workgroups still read the current one. With
    // ENG_G4_RESADD = 2 the adds run as their own launches instead.
    const bool fold = mxd::tunable("ENG_G4_RESADD", 1) != 2;
    float* xc = e->x;                 // the current residual
    float* xo = e->x2;                // the other buffer
    const float* pend_w = nullptr;    // a residual add pending on tmp (fold mode)
    float pend_post = 1.0f;
    // y (op)= W . [rmsnorm](x) after the pending add, if any.
    auto product = [&](const uint16_t* W, const float* norm_w, float* y, int M, int K, int epi,
                       const float* aux) -> int {
        if (!pend_w) {
            if (norm_w) return mxd_matvec_f16_rmsnorm(W, xc, norm_w, eps, 0, y, M, K, epi, aux, ms);
            return mxd_matvec_f16(W, xc, MXD_F32, y, M, K, epi, aux, ms);
        }
        const int r = mxd_matvec_f16_residual(W, xc, e->tmp, pend_w, pend_post, xo, norm_w, eps, 0, y, M, K, epi, aux,
                                              ms);
        std::swap(xc, xo);
        pend_w = nullptr;
        return r;
    };
    auto residual_add = [&](const float* w, float post) -> int {
        if (fold) {
            pend_w = w;
            pend_post = post;
            return MXD_OK;
        }
        return mxd_rmsnorm_add(e->tmp, w, xc, 1, D, eps, post, ms);
    };
    for (int l = 0; l < L; ++l) {
        const mxd_gemma4_layer& y = e->g4l[l];
        const LayerPtrs& Lp = e->L[l];
        const int hd = y.head_dim, F = y.ffn_dim;
        const bool own = owns_kv(e, l);
        if ((rc = product(Lp.wqkv, Lp.attn_norm, e->qkv, g4_qkv_dim(e, l), D, MXD_EPI_STORE, nullptr))) return rc;
        if ((rc = mxd_qk_norm_rope_kv(e->qkv, own ? Lp.kc : nullptr, own ? Lp.vc : nullptr, Lp.q_norm,
                                      own ? Lp.k_norm : nullptr, e->invf + (size_t)l * G4_FREQS, NH, own ? NKV : 0,
                                      hd, y.rope_pairs, e->max_ctx, eps, pos, 1, pos_dev, ms)))
            return rc;
        const int window = y.sliding ? c.window : 0;
        if (const int S = e->g4_splits[l]) {
            // the splits' partials, merged by the o projection as it loads them
            float* part = static_cast<float*>(e->attn_ws);
            if ((rc = mxd_attention_split_window(e->qkv, Lp.kc, Lp.vc, NH, NKV, hd, e->max_ctx, pos + 1, pos_dev,
                                                 window, 1.0f, S, part, e->attn_ws_bytes, ms)))
                return rc;
            if ((rc = mxd_matvec_f16_attn_merge_window(Lp.wo, part, S, NH, hd, e->max_ctx, pos + 1, pos_dev, window,
                                                       e->tmp, D, MXD_EPI_STORE, nullptr, ms)))
                return rc;
        } else {
            if ((rc = mxd_attention_window(e->qkv, Lp.kc, Lp.vc, e->att, NH, NKV, hd, e->max_ctx, pos + 1, pos_dev,
                                           window, 1.0f, e->attn_ws, e->attn_ws_bytes, ms)))
                return rc;
            if ((rc = mxd_matvec_f16(Lp.wo, e->att, MXD_F32, e->tmp, D, NH * hd, MXD_EPI_STORE, nullptr, ms)))
                return rc;
        }
        if ((rc = residual_add(Lp.post_attn_norm, 1.0f))) return rc;
        if (pend_w) {
            rc = mxd_gate_up_residual(Lp.wgate, Lp.wup, xc, e->tmp, pend_w, pend_post, xo, Lp.ffn_norm, eps, 0, e->h,
                                      F, D, MXD_ACT_GELU_TANH, ms);
            std::swap(xc, xo);
            pend_w = nullptr;
        } else {
            rc = mxd_gate_up_rmsnorm(Lp.wgate, Lp.wup, xc, Lp.ffn_norm, eps, 0, e->h, F, D, MXD_ACT_GELU_TANH, ms);
        }
        if (rc) return rc;
        if ((rc = mxd_matvec_f16(Lp.wdown, e->h, MXD_F32, e->tmp, D, F, MXD_EPI_STORE, nullptr, ms))) return rc;
        if ((rc = residual_add(Lp.post_ffn_norm, 1.0f))) return rc;
        if ((rc = product(Lp.ple_gate, nullptr, e->pleg, P, D, MXD_EPI_GELU_MUL, e->ple + (size_t)l * P))) return rc;
        if ((rc = mxd_matvec_f16(Lp.ple_out, e->pleg, MXD_F32, e->tmp, D, P, MXD_EPI_STORE, nullptr, ms))) return rc;
        if ((rc = residual_add(Lp.post_ple_norm, y.layer_scalar))) return rc;
    }
    if (!sample) return MXD_OK;
    // tied LM head; argmax on the raw logits (the softcap is monotonic, KG/main.swift:378-391)
    if ((rc = product(e->embed, e->final_norm, e->logits, V, D, MXD_EPI_STORE, nullptr))) return rc;
    return mxd::argmax_dev(e->logits, e->tokens, V, pos + 1, pos_dev, pos_dev != nullptr, e->am_ws, s,
                           pos_dev ? e->htokens_dev : nullptr);
}

namespace {

// The batched prefill of tokens[pos0 .. pos0 + T) (encodePrefillChunk,
// KG/main.swift:486-520): activations rounded to fp16 where the reference's
// chunk rounds them (the products round fp32 rows as they load them), the
// row-batched norms, q/k/v norm + RoPE + append and sliding-window causal
// attention; with sample, the last row takes the decode path's LM head and
// argmax into tokens[pos0 + T].
int g4_prefill_chunk(mxd_engine* e, int pos0, int T, bool sample) {
    const mxd_gemma4_config& c = e->g4;
    hipStream_t s = e->stream;
    mxd_stream_t ms = reinterpret_cast<mxd_stream_t>(s);
    const int D = c.dim, NH = c.n_heads, NKV = c.n_kv_heads, P = c.ple_dim, L = c.n_layers, V = c.vocab;
    const int LP = L * P;
    const float eps = c.rms_eps;
    void* ws = e->gm_ws;
    const size_t wsb = e->gm_ws_bytes;
    int rc;
    if ((rc = mxd::embed_dev(e->embed, e->tokens, pos0, nullptr, T, e->bx, D, sqrtf((float)D), V, s))) return rc;
    if ((rc = mxd::embed_dev(e->ple_embed, e->tokens, pos0, nullptr, T, e->bple, LP, sqrtf((float)P), c.ple_vocab, s)))
        return rc;
    if ((rc = mxd_gemm_f16(e->ple_proj, e->bx, MXD_F32, e->bpleproj, T, LP, D, MXD_EPI_STORE, ws, wsb, ms))) return rc;
    if ((rc = mxd_ple_combine(e->bpleproj, e->bple, e->ple_norm, T, L, P, 1.0f / sqrtf((float)D), eps, ms))) return rc;
    for (int l = 0; l < L; ++l) {
        const mxd_gemma4_layer& y = e->g4l[l];
        const LayerPtrs& Lp = e->L[l];
        const int hd = y.head_dim, F = y.ffn_dim, QKV = g4_qkv_dim(e, l), QD = g4_q_dim(e, l);
        const bool own = owns_kv(e, l);
        if ((rc = mxd_rmsnorm(e->bx, Lp.attn_norm, e->bxn, MXD_F16, T, D, eps, 0, ms))) return rc;
        if ((rc = mxd_gemm_f16(Lp.wqkv, e->bxn, MXD_F16, e->bqkv, T, QKV, D, MXD_EPI_STORE, ws, wsb, ms))) return rc;
        if ((rc = mxd_qk_norm_rope_kv(e->bqkv, own ? Lp.kc : nullptr, own ? Lp.vc : nullptr, Lp.q_norm,
                                      own ? Lp.k_norm : nullptr, e->invf + (size_t)l * G4_FREQS, NH, own ? NKV : 0,
                                      hd, y.rope_pairs, e->max_ctx, eps, pos0, T, nullptr, ms)))
            return rc;
        // attention and hidden rows rounded to fp16 where they are written, in
        // the fp32 buffers' memory (the o and down products stage fp16 rows)
        uint16_t* batt_h = reinterpret_cast<uint16_t*>(e->batt);
        if ((rc = mxd::attention_prefill_h16(e->bqkv, QKV, Lp.kc, Lp.vc, batt_h, QD, NH, NKV, hd, e->max_ctx, pos0, T,
                                             y.sliding ? c.window : 0, 1.0f, s)))
            return rc;
        if ((rc = mxd_gemm_f16(Lp.wo, batt_h, MXD_F16, e->btmp, T, D, QD, MXD_EPI_STORE, ws, wsb, ms))) return rc;
        if ((rc = mxd_rmsnorm_add(e->btmp, Lp.post_attn_norm, e->bx, T, D, eps, 1.0f, ms))) return rc;
        if ((rc = mxd_rmsnorm(e->bx, Lp.ffn_norm, e->bxn, MXD_F16, T, D, eps, 0, ms))) return rc;
        if (mxd::gemm_on_matrix_cores(T, D)) {
            uint16_t* bh_h = reinterpret_cast<uint16_t*>(e->bh);
            if ((rc = mxd::gemm_gate_up_f16_h16(Lp.wgate, Lp.wup, e->bxn, bh_h, T, F, D, MXD_ACT_GELU_TANH, ws, wsb, s)))
                return rc;
            if ((rc = mxd_gemm_f16(Lp.wdown, bh_h, MXD_F16, e->btmp, T, D, F, MXD_EPI_STORE, ws, wsb, ms))) return rc;
        } else {  // per-row matvecs: fp32 hidden rows, rounded as the down product loads them
            if ((rc = mxd_gemm_gate_up_f16(Lp.wgate, Lp.wup, e->bxn, e->bh, T, F, D, MXD_ACT_GELU_TANH, ws, wsb, ms)))
                return rc;
            if ((rc = mxd_gemm_f16(Lp.wdown, e->bh, MXD_F32, e->btmp, T, D, F, MXD_EPI_STORE, ws, wsb, ms))) return rc;
        }
        if ((rc = mxd_rmsnorm_add(e->btmp, Lp.post_ffn_norm, e->bx, T, D, eps, 1.0f, ms))) return rc;
        // the gate reads the un-normalized residual, rounded to fp16 (KG/main.swift:507)
        if ((rc = mxd_gemm_f16(Lp.ple_gate, e->bx, MXD_F32, e->bpleg, T, P, D, MXD_EPI_STORE, ws, wsb, ms))) return rc;
        if ((rc = mxd_ple_gate_act(e->bpleg, e->bple + (size_t)l * P, e->bpleg16, T, P, LP, ms))) return rc;
        if ((rc = mxd_gemm_f16(Lp.ple_out, e->bpleg16, MXD_F16, e->btmp, T, D, P, MXD_EPI_STORE, ws, wsb, ms)))
            return rc;
        if ((rc = mxd_rmsnorm_add(e->btmp, Lp.post_ple_norm, e->bx, T, D, eps, y.layer_scalar, ms))) return rc;
    }
    if (!sample) return MXD_OK;
    // Only the last row needs logits: it takes the decode path's head.
    HIP_OK(hipMemcpyAsync(e->x, e->bx + (size_t)(T - 1) * D, (size_t)D * 4, hipMemcpyDeviceToDevice, s),
           "mxd_engine_prefill");
    if ((rc = mxd_matvec_f16_rmsnorm(e->embed, e->x, e->final_norm, eps, 0, e->logits, V, D, MXD_EPI_STORE, nullptr,
                                     ms)))
        return rc;
    return mxd::argmax_dev(e->logits, e->tokens, V, pos0 + T, nullptr, false, e->am_ws, s);
}

// Split-K workspace of the chunk products for any chunk of 1 .. rows rows.
size_t g4_prefill_ws_bytes(const mxd_engine* e, int rows) {
    const mxd_gemma4_config& c = e->g4;
    const int D = c.dim, P = c.ple_dim, LP = c.n_layers * c.ple_dim;
    size_t m = 0;
    for (int T = 1; T <= rows; ++T) {
        m = max(m, mxd_gemm_f16_workspace_size(T, LP, D));
        m = max(m, mxd_gemm_f16_workspace_size(T, P, D));
        m = max(m, mxd_gemm_f16_workspace_size(T, D, P));
        for (int l = 0; l < c.n_layers; ++l) {
            const int F = e->g4l[l].ffn_dim;
            m = max(m, mxd_gemm_f16_workspace_size(T, g4_qkv_dim(e, l), D));
            m = max(m, mxd_gemm_f16_workspace_size(T, D, g4_q_dim(e, l)));
            m = max(m, mxd_gemm_gate_up_f16_workspace_size(T, F, D));
            m = max(m, mxd_gemm_f16_workspace_size(T, D, F));
        }
    }
    return m;
}

}  // namespace

int mxd_eng::g4_prefill(mxd_engine* e, int n) {
    if (n > 1 && mxd::tunable("ENG_NO_GEMM", 0) != 1) {
        for (int done = 0; done < n;) {
            const int rows = min(e->max_rows, n - done);
            if (int rc = g4_prefill_chunk(e, done, rows, done + rows == n)) return rc;
            done += rows;
        }
        return MXD_OK;
    }
    // Token by token through the decode step (the reference's --no-gemm
    // prefill, KG/main.swift:440-445).
    for (int p = 0; p < n; ++p)
        if (int rc = g4_step(e, p, nullptr, p == n - 1)) return rc;
    return MXD_OK;
}

extern "C" int mxd_engine_create_gemma4(const mxd_gemma4_config* cfg, int max_ctx, mxd_engine** out) {
    MXD_REQUIRE(out, MXD_ERR_INVALID_ARG, "mxd_engine_create_gemma4: null out");
    *out = nullptr;
    if (int rc = g4_check(cfg, max_ctx)) return rc;
    mxd_engine* e = new mxd_engine();
    e->arch = ENG_GEMMA4;
    e->g4 = *cfg;
    e->g4l.assign(cfg->layers, cfg->layers + cfg->n_layers);
    e->g4.layers = nullptr;  // the copy in g4l is the one kept
    e->max_ctx = max_ctx;
    mxd_model_config& mc = e->c;  // the fields the shared calls read
    mc.n_layers = cfg->n_layers;
    mc.dim = cfg->dim;
    mc.n_heads = cfg->n_heads;
    mc.n_kv_heads = cfg->n_kv_heads;
    mc.vocab = cfg->vocab;
    mc.rms_eps = cfg->rms_eps;
    const mxd_gemma4_config& c = e->g4;
    g4_plan(e);

    const int L = c.n_layers, NH = c.n_heads, NKV = c.n_kv_heads;
    const size_t D = c.dim, P = c.ple_dim, LP = (size_t)L * P;
    int max_qkv = 0, max_q = 0, max_f = 0;
    e->attn_ws_bytes = 0;
    // The decode attention leaves its splits' partials for the o projection
    // to merge when a layer sees at most 8 x 4 blocks (one 32-key block per
    // wave, 2 to 8 splits; ENG_ATT_FOLD = 2: never), as the Gemma-2B step
    // does, with at least ENG_ATT_SPLITS (default 6) splits (E2B at max_ctx
    // 384: 541-542 tok/s against 537); sliding layers see at most
    // window + 32 keys of the cache.
    e->g4_splits.assign(L, 0);
    for (int l = 0; l < L; ++l) {
        const mxd_gemma4_layer& y = e->g4l[l];
        max_qkv = max(max_qkv, g4_qkv_dim(e, l));
        max_q = max(max_q, g4_q_dim(e, l));
        max_f = max(max_f, y.ffn_dim);
        e->attn_ws_bytes = max(e->attn_ws_bytes, mxd_attention_workspace_size(NH, NKV, y.head_dim, max_ctx));
        const int keys = y.sliding && c.window > 0 ? min(max_ctx, c.window + 32) : max_ctx;
        int S = ((keys + 31) / 32 + 3) / 4;
        if (S >= 2 && S <= 8) S = max(S, min(8, mxd::tunable("ENG_ATT_SPLITS", 6)));
        if (S >= 2 && S <= 8 && mxd::tunable("ENG_ATT_FOLD", 1) != 2) {
            e->g4_splits[l] = S;
            e->attn_ws_bytes = max(e->attn_ws_bytes, (size_t)S * NH * (y.head_dim + 2) * sizeof(float));
        }
    }
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t o_x = take(D * 4), o_x2 = take(D * 4), o_tmp = take(D * 4), o_qkv = take((size_t)max_qkv * 4);
    const size_t o_att = take((size_t)max_q * 4), o_h = take((size_t)max_f * 4), o_logits = take((size_t)c.vocab * 4);
    const size_t o_ple = take(LP * 4), o_pleproj = take(LP * 4), o_pleg = take(P * 4);
    const size_t o_invf = take((size_t)L * G4_FREQS * 4), o_tok = take(((size_t)max_ctx + 1) * 4), o_pos = take(4);
    const size_t o_aws = take(e->attn_ws_bytes), o_am = take(mxd_argmax_workspace_size(c.vocab)), o_step = take(4);
    // prefill chunk buffers
    const size_t B = (size_t)(e->max_rows = min(prefill_rows(), max_ctx));
    e->gm_ws_bytes = g4_prefill_ws_bytes(e, e->max_rows);
    const size_t o_bx = take(B * D * 4), o_bxn = take(B * D * 2), o_bqkv = take(B * max_qkv * 4);
    const size_t o_batt = take(B * max_q * 4), o_bh = take(B * max_f * 4), o_btmp = take(B * D * 4);
    const size_t o_bple = take(B * LP * 4), o_bpleproj = take(B * LP * 4), o_bpleg = take(B * P * 4);
    const size_t o_bpleg16 = take(B * P * 2), o_gws = take(max(e->gm_ws_bytes, (size_t)16));
    std::vector<size_t> o_kc(L, 0), o_vc(L, 0);
    for (int l = 0; l < L; ++l) {
        if (!owns_kv(e, l)) continue;
        const size_t kv_bytes = (size_t)NKV * max_ctx * e->g4l[l].head_dim * 2;
        o_kc[l] = take(kv_bytes);
        o_vc[l] = take(kv_bytes);
    }
    e->abytes = off;
    if (int rc = allocate(e)) return rc;

    char* a = e->abase;
    e->x = reinterpret_cast<float*>(a + o_x);
    e->x2 = reinterpret_cast<float*>(a + o_x2);
    e->tmp = reinterpret_cast<float*>(a + o_tmp);
    e->qkv = reinterpret_cast<float*>(a + o_qkv);
    e->att = reinterpret_cast<float*>(a + o_att);
    e->h = reinterpret_cast<float*>(a + o_h);
    e->logits = reinterpret_cast<float*>(a + o_logits);
    e->ple = reinterpret_cast<float*>(a + o_ple);
    e->pleproj = reinterpret_cast<float*>(a + o_pleproj);
    e->pleg = reinterpret_cast<float*>(a + o_pleg);
    e->invf = reinterpret_cast<float*>(a + o_invf);
    e->tokens = reinterpret_cast<int32_t*>(a + o_tok);
    e->pos = reinterpret_cast<int32_t*>(a + o_pos);
    e->attn_ws = a + o_aws;
    e->am_ws = a + o_am;
    e->step = reinterpret_cast<int32_t*>(a + o_step);
    e->bx = reinterpret_cast<float*>(a + o_bx);
    e->bxn = reinterpret_cast<uint16_t*>(a + o_bxn);
    e->bqkv = reinterpret_cast<float*>(a + o_bqkv);
    e->batt = reinterpret_cast<float*>(a + o_batt);
    e->bh = reinterpret_cast<float*>(a + o_bh);
    e->btmp = reinterpret_cast<float*>(a + o_btmp);
    e->bple = reinterpret_cast<float*>(a + o_bple);
    e->bpleproj = reinterpret_cast<float*>(a + o_bpleproj);
    e->bpleg = reinterpret_cast<float*>(a + o_bpleg);
    e->bpleg16 = reinterpret_cast<uint16_t*>(a + o_bpleg16);
    e->gm_ws = a + o_gws;
    e->embed = wptr<uint16_t>(e, "embed");
    e->head = e->embed;
    e->final_norm = wptr<float>(e, "final_norm");
    e->ple_embed = wptr<uint16_t>(e, "ple_embed");
    e->ple_proj = wptr<uint16_t>(e, "ple_proj");
    e->ple_norm = wptr<float>(e, "ple_norm");
    e->L.resize(L);
    for (int l = 0; l < L; ++l) {
        const std::string p = "l" + std::to_string(l) + ".";
        LayerPtrs& Lp = e->L[l];
        Lp.attn_norm = wptr<float>(e, p + "attn_norm");
        Lp.ffn_norm = wptr<float>(e, p + "ffn_norm");
        Lp.wqkv = wptr<uint16_t>(e, p + "wqkv");
        Lp.wo = wptr<uint16_t>(e, p + "wo");
        Lp.wgate = wptr<uint16_t>(e, p + "wgate");
        Lp.wup = wptr<uint16_t>(e, p + "wup");
        Lp.wdown = wptr<uint16_t>(e, p + "wdown");
        Lp.q_norm = wptr<float>(e, p + "q_norm");
        Lp.k_norm = owns_kv(e, l) ? wptr<float>(e, p + "k_norm") : nullptr;
        Lp.post_attn_norm = wptr<float>(e, p + "post_attn_norm");
        Lp.post_ffn_norm = wptr<float>(e, p + "post_ffn_norm");
        Lp.post_ple_norm = wptr<float>(e, p + "post_ple_norm");
        Lp.ple_gate = wptr<uint16_t>(e, p + "ple_gate");
        Lp.ple_out = wptr<uint16_t>(e, p + "ple_out");
        const int src = e->g4l[l].kv_layer;
        Lp.kc = reinterpret_cast<uint16_t*>(a + o_kc[src]);
        Lp.vc = reinterpret_cast<uint16_t*>(a + o_vc[src]);
    }
    // Inverse frequencies theta^(-2i/hd) in double, stored as float, for the
    // rotated pairs and 0 (no rotation) past them (KG/main.swift:95-99).
    std::vector<float> invf((size_t)L * G4_FREQS, 0.0f);
    for (int l = 0; l < L; ++l) {
        const mxd_gemma4_layer& y = e->g4l[l];
        for (int i = 0; i < y.rope_pairs; ++i)
            invf[(size_t)l * G4_FREQS + i] =
                (float)(1.0 / pow((double)y.rope_theta, (double)(2 * i) / (double)y.head_dim));
    }
    hipError_t he = hipMemcpyAsync(e->invf, invf.data(), invf.size() * 4, hipMemcpyHostToDevice, e->stream);
    if (he == hipSuccess) he = hipStreamSynchronize(e->stream);
    if (he != hipSuccess) {
        destroy(e);
        return mxd::fail(MXD_ERR_HIP, "mxd_engine_create_gemma4: %s", hipGetErrorString(he));
    }
    *out = e;
    return MXD_OK;
}
