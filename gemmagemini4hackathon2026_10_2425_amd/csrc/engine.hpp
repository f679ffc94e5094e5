// The decode engine's state, shared by the Llama / Gemma step (engine.hip) and
// the Gemma-4 step (engine_gemma4.hip): one handle type serves both, so every
// mxd_engine_* call works on either.
#pragma once

#include "internal.hpp"

#include <string>
#include <unordered_map>
#include <vector>

namespace mxd_eng {

struct TensorInfo {
    std::string name;
    size_t offset, bytes;
    int dtype;  // MXD_F16 / MXD_F32
    uint64_t id;
    float shift = 0.0f;  // synthetic values are N(0, s^2) + shift (Gemma-4 norms: 1)
};

struct LayerPtrs {
    float *attn_norm, *ffn_norm;
    uint16_t *wqkv, *wo, *wgate, *wup, *wdown;
    uint16_t *kc, *vc;  // the caches the layer reads (a Gemma-4 shared layer: another layer's)
    // Gemma-4
    float *q_norm = nullptr, *k_norm = nullptr, *post_attn_norm = nullptr, *post_ffn_norm = nullptr,
          *post_ple_norm = nullptr;
    uint16_t *ple_gate = nullptr, *ple_out = nullptr;
};

inline size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Prompt rows per prefill chunk: the ENG_PREFILL_ROWS tunable (16 .. 4096),
// default 1024. Longer chunks keep more activation rows per weight tile on
// the matrix cores (Gemma-2B, measured on MI355X: pp512 66k tok/s as two
// 256-row chunks, 78k as one; pp1024 66k, 78k and 86k with 256-, 512- and
// 1024-row chunks).
inline int prefill_rows() { return max(16, min(4096, mxd::tunable("ENG_PREFILL_ROWS", 1024))); }

}  // namespace mxd_eng

#define HIP_OK(expr, what)                                                                         \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) return mxd::fail(MXD_ERR_HIP, "%s: %s", what, hipGetErrorString(e_)); \
    } while (0)

enum { ENG_LLAMA = 0, ENG_GEMMA4 = 1 };

struct mxd_engine {
    int arch = ENG_LLAMA;
    // Llama / Gemma shape; for Gemma-4 only n_layers, dim, n_heads,
    // n_kv_heads, vocab and rms_eps are set (the rest lives in g4 / g4l).
    mxd_model_config c{};
    int max_ctx = 0;
    hipStream_t stream = nullptr;
    std::vector<mxd_eng::TensorInfo> tensors;
    std::unordered_map<std::string, int> index;
    char* wbase = nullptr;
    size_t wbytes = 0;
    char* abase = nullptr;
    size_t abytes = 0;
    std::vector<mxd_eng::LayerPtrs> L;
    uint16_t* embed = nullptr;
    uint16_t* head = nullptr;  // the LM head: embed (tied) or lm_head
    float* final_norm = nullptr;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
    float* invf = nullptr;
    int32_t *tokens = nullptr, *pos = nullptr;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    // Splits of the decode attention when its merge is folded into the o
    // projection (one 32-key block per wave at max_ctx); 0 = the separate
    // attention with its own merge.
    int att_splits = 0;
    void* am_ws = nullptr;
    hipGraphExec_t graph = nullptr;
    // Streaming decode: the captured step's argmax also writes each token to
    // pinned host memory (htokens, its device view htokens_dev), and every
    // replayed step records an event in a ring indexed by its position, so a
    // caller waits for one step without draining the ones queued after it.
    int32_t* htokens = nullptr;
    int32_t* htokens_dev = nullptr;
    static constexpr int RING = 16;
    hipEvent_t step_done[RING] = {};
    // The position the last decode run left in the device counter (-1: not
    // known), so a run that continues from it needs no counter write.
    int pos_next = -1;
    // The fused attention half of each layer (attn_block): its workspace of
    // tagged words, the step counter its tags come from (advanced by the
    // embedding kernel of every step) and its error word.
    bool fused = false;
    void* ab_ws = nullptr;
    size_t ab_ws_bytes = 0;
    int32_t* step = nullptr;
    int* ab_err = nullptr;
    // prefill chunk buffers: rows x {dim f32, dim f16, qkv f32, q f32, ffn f32}
    // (the products round fp32 rows to fp16 as they load them), and the
    // products' split-K workspace
    int max_rows = 0;
    float *bx = nullptr, *bqkv = nullptr, *batt = nullptr, *bh = nullptr;
    uint16_t* bxn = nullptr;
    void* gm_ws = nullptr;
    size_t gm_ws_bytes = 0;

    // Gemma-4: model facts, the per-layer-embedding tables and buffers (ple:
    // [n_layers][ple_dim] per row, pleproj the same, pleg [ple_dim]), the
    // residual branch buffer tmp [dim], and the prefill chunk's counterparts.
    mxd_gemma4_config g4{};
    std::vector<mxd_gemma4_layer> g4l;
    uint16_t *ple_embed = nullptr, *ple_proj = nullptr;
    float* ple_norm = nullptr;
    float *tmp = nullptr, *ple = nullptr, *pleproj = nullptr, *pleg = nullptr;
    float* x2 = nullptr;  // the second residual buffer (x and x2 alternate)
    // per layer: splits of the attention whose partials the o projection
    // merges (0: the attention with its own output, then the o projection)
    std::vector<int> g4_splits;
    float *btmp = nullptr, *bple = nullptr, *bpleproj = nullptr, *bpleg = nullptr;
    uint16_t* bpleg16 = nullptr;

    int qkv_dim() const { return (c.n_heads + 2 * c.n_kv_heads) * c.head_dim; }
    int q_dim() const { return c.n_heads * c.head_dim; }
};

namespace mxd_eng {

inline void add_tensor(mxd_engine* e, const std::string& name, size_t elems, int dtype, uint64_t id, size_t& off,
                       float shift = 0.0f) {
    const size_t bytes = elems * (dtype == MXD_F32 ? 4 : 2);
    e->index[name] = (int)e->tensors.size();
    e->tensors.push_back({name, off, bytes, dtype, id, shift});
    off += align256(bytes);
}

template <typename T>
T* wptr(mxd_engine* e, const std::string& name) {
    return reinterpret_cast<T*>(e->wbase + e->tensors[e->index.at(name)].offset);
}

inline void destroy(mxd_engine* e) {
    if (!e) return;
    if (e->graph) (void)hipGraphExecDestroy(e->graph);
    for (hipEvent_t& ev : e->step_done)
        if (ev) (void)hipEventDestroy(ev);
    if (e->htokens) (void)hipHostFree(e->htokens);
    if (e->wbase) (void)hipFree(e->wbase);
    if (e->abase) (void)hipFree(e->abase);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

// Stream, arenas (weights wbytes, buffers abytes), pinned token mirror and
// step events of a planned engine; destroys e on failure.
int allocate(mxd_engine* e);

// Gemma-4 (engine_gemma4.hip): one decode step, and a prefill of tokens[0..n).
int g4_step(mxd_engine* e, int pos, int32_t* pos_dev, bool sample);
int g4_prefill(mxd_engine* e, int n);

}  // namespace mxd_eng
