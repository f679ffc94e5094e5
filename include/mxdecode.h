/*
 * mxdecode.h — C ABI of libmxdecode, the MI355X (gfx950) LLM decode hot path.
 *
 * Every entry point:
 *   - takes caller-owned DEVICE pointers and plain sizes (no framework types),
 *   - enqueues work on `stream` (a hipStream_t passed as void*; NULL = the null
 *     stream) and returns without synchronising,
 *   - returns MXD_OK (0) or a negative MXD_ERR_* code and never aborts; the text
 *     of the last failure on the calling thread is mxd_last_error().
 * Argument checks happen on the host before anything is launched, so a bad
 * shape never reaches the GPU.
 *
 * Each declaration names the reference interface it replaces. The reference is
 * a Metal/Swift engine whose device operators are Metal kernels bound by
 * buffer index; paths below are relative to ios_kernels/kernels/:
 *   KL = unsloth__Llama-3.2-1B-Instruct/kernel_metal_f16_20261024-1620/
 *   KG = google__gemma-4-E2B-it/kernel_metal_f16_20261025-1225/
 *
 * Storage conventions (as in the reference, KL/kernels.metal:7-10):
 *   weights fp16 row-major [out_features][in_features]; activations and the
 *   residual stream fp32; KV cache fp16. fp16 values travel as uint16_t bits.
 * KV cache layout (this library's contract). Each cache holds n_kv_heads *
 * max_ctx * head_dim fp16 values (the size of the reference's
 * [kv_head][max_ctx][head_dim], KL/kernels.metal:10), max_ctx % 32 == 0,
 * cut into tiles of 32 positions; the tile of position p of kv head h starts
 * at element (h * max_ctx + (p & ~31)) * head_dim. Inside a tile, with
 * k = p & 31 and d the dim, values sit in the order the attention kernel's
 * matrix-core operands are loaded, so every operand is one contiguous 1 KiB
 * wave load:
 *   K: ((t * head_dim/32 + c) * 64 + g * 16 + col) * 8 + e
 *      t = (k >> 2) & 1, col = ((k >> 3) << 2) | (k & 3),
 *      c = d >> 5, g = (d >> 3) & 3, e = d & 7
 *   V: ((d >> 4) * 64 + (k >> 3) * 16 + (d & 15)) * 8 + (k & 7)
 */
#ifndef MXDECODE_H
#define MXDECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mxd_stream_t;

enum {
    MXD_OK = 0,
    MXD_ERR_INVALID_ARG = -1,    /* null pointer, negative size, unknown enum */
    MXD_ERR_UNSUPPORTED = -2,    /* shape/alignment the kernels do not handle */
    MXD_ERR_HIP = -3,            /* a HIP runtime call or launch failed       */
    MXD_ERR_WORKSPACE = -4,      /* workspace missing or too small            */
    MXD_ERR_ALLOC = -5           /* device allocation failed                  */
};

enum { MXD_F32 = 0, MXD_F16 = 1 };                               /* activation dtypes */
enum { MXD_W_F16 = 0, MXD_W_Q8B32 = 1 };                         /* weight formats    */
enum { MXD_EPI_STORE = 0, MXD_EPI_ADD = 1, MXD_EPI_GELU_MUL = 2 }; /* KG/kernels.metal:152-153 */
enum { MXD_ACT_GELU_TANH = 0, MXD_ACT_SILU = 1 };

/* ---- library ---------------------------------------------------------- */

/* Text of the last failure on this thread ("" if none). */
const char* mxd_last_error(void);
/* ABI version of this header (bumped on any signature change). */
int mxd_abi_version(void);
/* Kernel tunables by name, e.g. "MV_NR" (rows per workgroup) or "MV_NW"
 * (waves splitting K). value <= 0 restores the shape-based default.
 * Replaces the reference's `--define NAME=VALUE` (KL/main.swift:178-184). */
int mxd_set_tunable(const char* name, int value);

/* ---- synthetic weights -------------------------------------------------- */

/* dst[i] = N(0, stddev^2)-distributed value for element i of tensor
 * (seed, tensor_id), from a counter-based hash (splitmix64) summed over
 * eight 16-bit uniforms and scaled in fp32; dtype MXD_F32 or MXD_F16 (RNE).
 * Stands in for the converted HF checkpoint (KL/convert_weights.py:71-89),
 * which needs a network fetch; the oracle computes the same bits on the CPU. */
int mxd_fill_normal(void* dst, int dtype, uint64_t n, uint64_t seed, uint64_t tensor_id,
                    float stddev, mxd_stream_t stream);

/* ---- matvec (GEMV) ------------------------------------------------------ */

/* y = W·x, W fp32 [M][K] row-major, x fp32 [K], y fp32 [M]. fp32 variant of
 * matvec_f16 (KL/kernels.metal:106-137) for the fp32 parity configuration. */
int mxd_gemv_f32(const float* W, const float* x, float* y, int M, int K, mxd_stream_t stream);

/* y (op)= W·x with W fp16 [M][K]; x fp32 or fp16 (x_dtype); y fp32; fp32
 * accumulation. epilogue: STORE y=s, ADD y+=s, GELU_MUL y=gelu_tanh(s)*aux.
 * Replaces matvec_f16 / matvec_f16_add / matvec_f16_gelu_mul
 * (KG/kernels.metal:159-198, KL/kernels.metal:106-137; host KG/main.swift:303-316).
 * Needs K % 8 == 0 (16-byte rows); any M. */
int mxd_matvec_f16(const uint16_t* W, const void* x, int x_dtype, float* y, int M, int K,
                   int epilogue, const float* aux, mxd_stream_t stream);

/* Same contract with int8 block-32 weights: y[r] = sum_b s[r][b] * sum_{k in b} q[r][k]*x[k].
 * Wq int8 [M][K]; scales fp16 [M][K/32] (= max|w|/127 of the block).
 * No reference counterpart (Q8_0 is a roadmap item, ios_kernels/PLAN.md:175);
 * drops in wherever matvec_f16 is bound. Needs K % 32 == 0. */
int mxd_matvec_q8b32(const int8_t* Wq, const uint16_t* scales, const void* x, int x_dtype,
                     float* y, int M, int K, int epilogue, const float* aux, mxd_stream_t stream);

/* Fused gated up-projection h[r] = act(Wg[r]·x) * (Wu[r]·x), F rows, K columns.
 * w_format MXD_W_F16 (scales ignored) or MXD_W_Q8B32; x fp32 or fp16.
 * Replaces matvec_gate_up_gelu (KG/kernels.metal:205-234) and
 * matvec_gate_up_silu (KL/kernels.metal:144-173); host KG/main.swift:318-330. */
int mxd_matvec_gate_up(int w_format, const void* Wg, const uint16_t* sg, const void* Wu,
                       const uint16_t* su, const void* x, int x_dtype, float* h, int F, int K,
                       int act, mxd_stream_t stream);

/* ---- fused decode-step operators ------------------------------------------- */

/* y (op)= W · rmsnorm(x): the RMSNorm (KL/kernels.metal:71-96, weight w or
 * 1 + w) folded into the matvec's activation loads; W fp16 [M][K], x and y fp32.
 * Fuses the reference's rmsnorm_f32 + matvec_f16 pair (KL/main.swift:333-334). */
int mxd_matvec_f16_rmsnorm(const uint16_t* W, const float* x, const float* norm_w, float eps, int plus_one,
                           float* y, int M, int K, int epilogue, const float* aux, mxd_stream_t stream);

/* h = act(Wg · rmsnorm(x)) * (Wu · rmsnorm(x)); fuses rmsnorm_f32 +
 * matvec_gate_up_* (KL/main.swift:338-339, KG/kernels.metal:205-234). */
int mxd_gate_up_rmsnorm(const uint16_t* Wg, const uint16_t* Wu, const float* x, const float* norm_w, float eps,
                        int plus_one, float* h, int F, int K, int act, mxd_stream_t stream);

/* The same products after a sandwich norm's residual add: with
 * x' = (x + res_src * rsqrt(mean(res_src^2) + eps) * res_w) * res_post (the
 * mxd_rmsnorm_add of res_src into x), y (op)= W · rmsnorm(x') (norm_w NULL:
 * W · x'), or h = act(Wg · rmsnorm(x')) * (Wu · rmsnorm(x')). Every
 * workgroup forms x' itself; one of them writes it to x_out, which must not
 * alias x or res_src (x' is the next residual). Fuses Gemma-4's rmsnorm_add
 * into the product that follows it (KG/main.swift:405-422). */
int mxd_matvec_f16_residual(const uint16_t* W, const float* x, const float* res_src, const float* res_w,
                            float res_post, float* x_out, const float* norm_w, float eps, int plus_one, float* y,
                            int M, int K, int epilogue, const float* aux, mxd_stream_t stream);
int mxd_gate_up_residual(const uint16_t* Wg, const uint16_t* Wu, const float* x, const float* res_src,
                         const float* res_w, float res_post, float* x_out, const float* norm_w, float eps,
                         int plus_one, float* h, int F, int K, int act, mxd_stream_t stream);

/* [q | k | v] = Wqkv · rmsnorm(x) (norm_w NULL: no norm), then RoPE on q and k
 * at pos and the K/V append, in the projection's epilogue: q (rotated, fp32,
 * n_heads*head_dim) goes to `q`, k and v (fp16) to the tiled caches. Fuses
 * rmsnorm_f32 + matvec_f16(wqkv) + rope_kv (KL/main.swift:333-335). With pos_dev
 * the position is read on the device. head_dim % 32 == 0, max_ctx % 32 == 0. */
int mxd_qkv_rope_kv(const uint16_t* Wqkv, const float* x, const float* norm_w, float eps, int plus_one, float* q,
                    uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads, int n_kv_heads,
                    int head_dim, int K, int max_ctx, int pos, const int32_t* pos_dev, mxd_stream_t stream);

/* y (op)= W · x where x is the single-query attention output given as the
 * unmerged partials of mxd_attention_split (n_splits <= 8): every workgroup
 * merges the x values it reads with the log-sum-exp rule, so the attention
 * needs no merge launch. W fp16 [M][n_heads*head_dim]; the active splits
 * follow from n_keys, or *n_keys_dev + 1, as in the producer. Fuses the
 * attention output into the output projection (KL/main.swift:336-337:
 * attention then matvec_add(wo)). */
int mxd_matvec_f16_attn_merge(const uint16_t* W, const float* partials, int n_splits, int n_heads,
                              int head_dim, int max_ctx, int n_keys, const int32_t* n_keys_dev, float* y,
                              int M, int epilogue, const float* aux, mxd_stream_t stream);
/* The merge of mxd_attention_split_window's partials (the same window). */
int mxd_matvec_f16_attn_merge_window(const uint16_t* W, const float* partials, int n_splits, int n_heads,
                                     int head_dim, int max_ctx, int n_keys, const int32_t* pos_dev, int window,
                                     float* y, int M, int epilogue, const float* aux, mxd_stream_t stream);

/* ---- normalisation, embedding, casts ------------------------------------ */

/* y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * (plus_one ? 1 + w : w), rows x D,
 * x fp32, w fp32, y fp32 or fp16 (y_dtype). Replaces rmsnorm_f32/rmsnorm_f16
 * (KL/kernels.metal:71-96; host KL/main.swift:233-244). plus_one selects the
 * Gemma (1 + w) weight convention. */
int mxd_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int rows, int D, float eps,
                int plus_one, mxd_stream_t stream);

/* x[r] += the sum of a product's K-split partials for row r (part: n_splits x
 * [rows][D], as mxd_gemm_q8b32_partials leaves them; summed in split order,
 * bit-identical to mxd_gemm_q8b32 with MXD_EPI_ADD), then y = rmsnorm(x) as
 * mxd_rmsnorm computes it. x, part, w 16-byte aligned. Fuses the residual
 * add of gemm_f16_add (KL/kernels.metal:389-441) with the rmsnorm that
 * follows it in the batched layer (KL/main.swift:422-428). */
int mxd_rmsnorm_residual_sum(float* x, const float* part, int n_splits, const float* w, void* y, int y_dtype,
                             int rows, int D, float eps, int plus_one, mxd_stream_t stream);

/* x[r][i] = float(E[tokens[pos + r]][i]) * scale for r < rows. Replaces embed
 * (KL/kernels.metal:31-39) and embed_rows (KG/kernels.metal:34-42); the token
 * index is read on the device, so a sampled token feeds the next step without
 * a host round trip (KL/main.swift:319-320). */
int mxd_embed(const uint16_t* E, const int32_t* tokens, int pos, int rows, float* x, int D,
              float scale, int vocab, mxd_stream_t stream);

/* dst = fp16(src), n elements. Replaces f32_to_f16 (KL/kernels.metal:361-365). */
int mxd_f32_to_f16(const float* src, uint16_t* dst, size_t n, mxd_stream_t stream);

/* ---- RoPE + KV-cache append --------------------------------------------- */

/* qkv rows are [q n_heads*hd | k n_kv_heads*hd | v n_kv_heads*hd] fp32 (row r at
 * position pos0 + r). Rotates q in place and k (HF rotate_half pairs (i, i+hd/2),
 * angle = pos * inv_freq[i] in fp32, accurate sin/cos), then appends fp16 k to
 * kcache and fp16 v to vcache at that position (tile layouts above).
 * head_dim % 32 == 0.
 * Replaces rope_kv (KL/kernels.metal:182-224; host KL/main.swift:275-287). */
int mxd_rope_kv(float* qkv, uint16_t* kcache, uint16_t* vcache, const float* inv_freq,
                int n_heads, int n_kv_heads, int head_dim, int max_ctx, int pos0, int rows,
                mxd_stream_t stream);

/* ---- single-query attention ---------------------------------------------- */

/* Workspace bytes mxd_attention needs for this shape (any max_ctx). */
size_t mxd_attention_workspace_size(int n_heads, int n_kv_heads, int head_dim, int max_ctx);

/* out[h] = softmax(scale * q[h]·K[kvh][0..n_keys)) · V[kvh][0..n_keys) for
 * every query head h, kvh = h / (n_heads / n_kv_heads) (GQA/MQA), fp32 scores
 * and softmax. Split over the key axis with an online softmax and a
 * log-sum-exp merge, so n_keys is bounded only by max_ctx; the G = n_heads /
 * n_kv_heads query heads of a group share each K/V tile. head_dim 64, 128, 256
 * or 512; max_ctx % 32 == 0. q [n_heads*hd] fp32, out [n_heads*hd] fp32.
 * If n_keys_dev is not NULL the key count is read on the device from
 * *n_keys_dev (+1), so a captured step replays at a moving position.
 * Replaces attention (KL/kernels.metal:235-305, KG/kernels.metal:317-399;
 * host KL/main.swift:289-303) for the decode case T = 1. */
int mxd_attention(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                  int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys,
                  const int32_t* n_keys_dev, float scale, void* workspace, size_t ws_bytes,
                  mxd_stream_t stream);

/* mxd_attention for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * kernels and arguments without the workspace; no reference counterpart. The
 * split partials live in a device array of mxd_attention_noalloc_max_scratch()
 * bytes (8 MiB) that the library holds on each GPU it runs on until the process
 * ends; a shape needing more returns MXD_ERR_UNSUPPORTED. The call allocates
 * nothing. Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (different streams, or threads) race: serialise them. */
size_t mxd_attention_noalloc_max_scratch(void);
int mxd_attention_noalloc(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                          int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys,
                          const int32_t* n_keys_dev, float scale, mxd_stream_t stream);

/* The split half of mxd_attention without its merge: split s of n_splits
 * (1 .. 512) takes the 32-key blocks s, s + n_splits, ... and writes its
 * unnormalised partial, O to partials[s][h][0..hd) and (max, sum) of its
 * log2-domain scores to partials[n_splits*n_heads*hd + (s*n_heads + h)*2 ..],
 * for the splits that hold a block (min(n_splits, ceil(n_keys / 32))); with
 * no keys, split 0 holds a zero partial (O = 0, max 0, sum 1). partial_bytes
 * >= n_splits*n_heads*(hd + 2)*4. The merge belongs to the consumer
 * (mxd_matvec_f16_attn_merge). Same shapes and caches as mxd_attention;
 * replaces the reference attention's per-head loop over keys
 * (KL/kernels.metal:258-304) for T = 1. */
int mxd_attention_split(const float* q, const uint16_t* kcache, const uint16_t* vcache, int n_heads,
                        int n_kv_heads, int head_dim, int max_ctx, int n_keys, const int32_t* n_keys_dev,
                        float scale, int n_splits, float* partials, size_t partial_bytes,
                        mxd_stream_t stream);
/* The same over a sliding window: the blocks dealt to the splits start at the
 * window's first block, and the active splits count the attended blocks
 * (min(n_splits, ceil(n_keys / 32) - start / 32), start = max(0, n_keys -
 * window)). Merge with mxd_matvec_f16_attn_merge_window at the same window. */
int mxd_attention_split_window(const float* q, const uint16_t* kcache, const uint16_t* vcache, int n_heads,
                               int n_kv_heads, int head_dim, int max_ctx, int n_keys, const int32_t* n_keys_dev,
                               int window, float scale, int n_splits, float* partials, size_t partial_bytes,
                               mxd_stream_t stream);

/* Causal attention of a prefill chunk: `rows` queries at positions pos0 ..
 * pos0 + rows - 1 (their keys and values already in the caches), query t over
 * keys [0, pos0 + t]. q rows are q_stride floats apart (a multiple of 4; the
 * q part of a qkv row works in place), out rows out_stride. Same head dims,
 * group sizes and cache layout as mxd_attention. Replaces attention with
 * T > 1 (KL/kernels.metal:245-305: n = pos0 + t + 1, q_row_stride; host
 * attention(enc, layer:, pos0:, rows:) in KL/main.swift:412-446). */
int mxd_attention_prefill(const float* q, int q_stride, const uint16_t* kcache, const uint16_t* vcache,
                          float* out, int out_stride, int n_heads, int n_kv_heads, int head_dim, int max_ctx,
                          int pos0, int rows, float scale, mxd_stream_t stream);

/* Sliding-window forms: a query that sees n keys attends to keys
 * [max(0, n - window), n) (window 0: all n). Gemma-4's sliding layers
 * (window 512; KG/kernels.metal:306-393, start = pos + 1 - window,
 * AttnParams.window; host KG/main.swift:358-376). Otherwise identical to
 * mxd_attention / mxd_attention_prefill, head_dim 512 included. */
int mxd_attention_window(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                         int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys,
                         const int32_t* n_keys_dev, int window, float scale, void* workspace, size_t ws_bytes,
                         mxd_stream_t stream);
int mxd_attention_prefill_window(const float* q, int q_stride, const uint16_t* kcache, const uint16_t* vcache,
                                 float* out, int out_stride, int n_heads, int n_kv_heads, int head_dim,
                                 int max_ctx, int pos0, int rows, int window, float scale, mxd_stream_t stream);

/* ---- Gemma-4 operators ---------------------------------------------------- */

/* Sandwich-norm residual update, per row r of D values:
 * x[r] = (x[r] + src[r] * rsqrt(mean(src[r]^2) + eps) * w) * post, fp32.
 * post is the layer scalar after a layer's last residual add, else 1.
 * Replaces rmsnorm_add (KG/kernels.metal:100-125; host KG/main.swift:273-285). */
int mxd_rmsnorm_add(const float* src, const float* w, float* x, int rows, int D, float eps, float post,
                    mxd_stream_t stream);

/* Per-layer-embedding combine, rows x n_layers slices of P values:
 * ple[r][l] = (rmsnorm(proj[r][l] * proj_scale) * w + ple[r][l]) / sqrt(2),
 * with ple holding the scaled token-identity rows on entry.
 * Replaces ple_combine (KG/kernels.metal:127-149; host KG/main.swift:287-299). */
int mxd_ple_combine(const float* proj, float* ple, const float* w, int rows, int n_layers, int P,
                    float proj_scale, float eps, mxd_stream_t stream);

/* Prefill's gate activation of the per-layer inputs: dst[t][i] =
 * fp16(gelu_tanh(src[t][i]) * ple[t * ple_stride + i]) for rows t, i < P (ple
 * points at the layer's slice of the per-layer-input rows). Replaces
 * ple_gate_act (KG/kernels.metal:451-461; host KG/main.swift:530-539). */
int mxd_ple_gate_act(const float* src, const float* ple, uint16_t* dst, int rows, int P, int ple_stride,
                     mxd_stream_t stream);

/* qkv rows [q n_heads*hd | k n_kv_heads*hd | v n_kv_heads*hd] fp32 (row r at
 * position pos0 + r, or *pos_dev + r): per-head RMSNorm of q (weight q_w),
 * k (k_w) and v (no weight), HF rotate_half RoPE on q and k over the rotation
 * pairs i < rope_pairs (the rest unrotated), q written back in place, k and
 * v appended as fp16 to the tiled caches. n_kv_heads 0: q only (a layer that
 * reads another layer's cache). head_dim a multiple of 32 up to 512.
 * Replaces qkv_norm_rope (KG/kernels.metal:236-304; host KG/main.swift:338-356). */
int mxd_qk_norm_rope_kv(float* qkv, uint16_t* kcache, uint16_t* vcache, const float* q_w, const float* k_w,
                        const float* inv_freq, int n_heads, int n_kv_heads, int head_dim, int rope_pairs,
                        int max_ctx, float eps, int pos0, int rows, const int32_t* pos_dev,
                        mxd_stream_t stream);

/* ---- greedy sample -------------------------------------------------------- */

/* Workspace bytes mxd_argmax needs for N logits. */
size_t mxd_argmax_workspace_size(int N);

/* tokens[out_idx] = argmax(logits[0..N)), ties to the lowest index.
 * Replaces argmax (KL/kernels.metal:310-345; host KL/main.swift:305-315). The
 * workspace must be zeroed once before first use; the kernel leaves it zeroed. */
int mxd_argmax(const float* logits, int32_t* tokens, int N, int out_idx, void* workspace,
               size_t ws_bytes, mxd_stream_t stream);

/* ---- ragged batch over a paged KV cache ----------------------------------------
 * The reference decodes one sequence over a contiguous cache and has no paging
 * or batching (ios_kernels/surfaces/DESIGN_AND_LIMITATIONS.md:48,87-88); these
 * entry points decode a batch of sequences of different lengths in one launch
 * per op.
 *
 * Page pool (per layer): n_pages pages of 16 positions of every kv head; the
 * (page, kv head) slab of 16 * head_dim fp16 values starts at element
 * (page * n_kv_heads + kvh) * 16 * head_dim and is stored in MFMA operand order
 * (one half of a 32-position tile of the contiguous layout, made contiguous):
 *   K: key r (0..15), dim d at ((((d >> 5) * 2 + ((r >> 2) & 1)) * 4 + ((d >> 3) & 3)) * 8 + rr) * 8 + (d & 7),
 *      rr = ((r >> 3) << 2) | (r & 3)
 *   V: key r, dim d at (((d >> 4) * 2 + (r >> 3)) * 16 + (d & 15)) * 8 + (r & 7)
 * page_table is int32 [n_seqs][max_pages]: entry [b][i] is the pool page that
 * holds positions 16i .. 16i + 15 of sequence b (any order; the pool is shared).
 * seq_lens is int32 [n_seqs]: the keys of sequence b after this step's append,
 * so its new token sits at position seq_lens[b] - 1. Row b of every activation
 * matrix belongs to sequence b. Device-side values are clamped so that a bad
 * table entry or length cannot address outside the pool or the table. */

/* Rotates q and k of row b of qkv [n_seqs][(n_heads + 2 n_kv_heads) head_dim]
 * in place at position seq_lens[b] - 1 and appends fp16 k and v there.
 * Replaces rope_kv (KL/kernels.metal:182-224) for a batch of sequences, each at
 * its own position, over the page pool. */
int mxd_rope_kv_paged(float* qkv, uint16_t* kpool, uint16_t* vpool, int n_pages, const float* inv_freq,
                      int n_heads, int n_kv_heads, int head_dim, const int32_t* page_table, int max_pages,
                      const int32_t* seq_lens, int n_seqs, mxd_stream_t stream);

/* mxd_rope_kv_paged fused with the sum of the q|k|v product's K-split
 * partials (part: n_splits x [n_seqs][(n_heads + 2 n_kv_heads) head_dim], as
 * mxd_gemm_q8b32_partials leaves them): each value is the partials' sum in
 * split order, bit-identical to mxd_gemm_q8b32's output, so the product needs
 * no summing launch. Only the q part of qkv is written (rotated), which is all
 * mxd_attention_paged reads of it. Fuses the reference's rope_kv
 * (KL/kernels.metal:182-224) with the sum it takes for granted. */
int mxd_rope_kv_paged_sum(const float* part, int n_splits, float* qkv, uint16_t* kpool, uint16_t* vpool,
                          int n_pages, const float* inv_freq, int n_heads, int n_kv_heads, int head_dim,
                          const int32_t* page_table, int max_pages, const int32_t* seq_lens, int n_seqs,
                          mxd_stream_t stream);

/* Workspace bytes mxd_attention_paged needs (max_keys bounds every seq_lens).
 * The size follows the schedule the call will use: up to 2048 sequences the
 * batch's (sequence, kv head, block) items are dealt evenly over the
 * workgroups resident on the GPU (partials per workgroup piece plus a block
 * prefix), beyond that a fixed number of splits per sequence; query it again
 * after changing the ATT_SCHED / ATT_SKWG / ATT_BPS tunables. */
size_t mxd_attention_paged_workspace_size(int n_heads, int n_kv_heads, int head_dim, int n_seqs, int max_keys);

/* out[b][h] = softmax(scale * q[b][h] · K_b[kvh]) · V_b[kvh] over the seq_lens[b]
 * keys of sequence b, for all sequences in one launch. q rows are q_stride
 * floats apart (the q part of a qkv row works in place), out rows out_stride.
 * Replaces attention (KL/kernels.metal:235-305) for a paged ragged batch; same
 * group sizes and head dims as mxd_attention. A sequence with no keys gets a
 * zero output. */
int mxd_attention_paged(const float* q, int q_stride, const uint16_t* kpool, const uint16_t* vpool, int n_pages,
                        const int32_t* page_table, int max_pages, const int32_t* seq_lens, int n_seqs, float* out,
                        int out_stride, int n_heads, int n_kv_heads, int head_dim, int max_keys, float scale,
                        void* workspace, size_t ws_bytes, mxd_stream_t stream);

/* Workspace bytes mxd_gemm_q8b32 needs (0 when it does not split K). */
size_t mxd_gemm_q8b32_workspace_size(int n_rows, int M, int K);

/* Y[b] (op)= dequant(Wq, scales) · X[b] for the n_rows rows of X ([n_rows][K],
 * x_dtype MXD_F16, or MXD_F32 rounded to nearest-even fp16 as it is loaded,
 * the rounding of mxd_f32_to_f16); Y fp32 [n_rows][M]; epilogue
 * MXD_EPI_STORE or MXD_EPI_ADD. From 16 rows on (and K % 128 == 0) this runs
 * on the matrix cores; below, one matvec per row. The batched-matrix
 * counterpart of gemm_f16 / gemm_f16_add (KL/kernels.metal:376-441), with
 * int8 block-32 weights; fp32 X folds the reference's f32_to_f16 cast
 * (KL/main.swift:448-454) into the product. */
int mxd_gemm_q8b32(const int8_t* Wq, const uint16_t* scales, const void* X, int x_dtype, float* Y,
                   int n_rows, int M, int K, int epilogue, void* workspace, size_t ws_bytes,
                   mxd_stream_t stream);

/* Bytes of the K-split partials mxd_gemm_q8b32_partials leaves (0 below 16
 * rows or when K % 128 != 0, where it does not apply). */
size_t mxd_gemm_q8b32_partials_size(int n_rows, int M, int K);

/* mxd_gemm_q8b32 (MXD_EPI_STORE) on the matrix cores with the K-split sum
 * left to the consumer: part receives *n_splits partial products
 * [n_splits][n_rows][M] (a single split is the product itself), which
 * mxd_rope_kv_paged_sum and mxd_rmsnorm_residual_sum add as they load them.
 * Needs n_rows >= 16 and K % 128 == 0. The reference's gemm_f16
 * (KL/kernels.metal:376-441) with its reduction deferred to the next op. */
int mxd_gemm_q8b32_partials(const int8_t* Wq, const uint16_t* scales, const void* X, int x_dtype, float* part,
                            size_t part_bytes, int n_rows, int M, int K, int* n_splits, mxd_stream_t stream);

/* Workspace bytes mxd_gemm_gate_up_q8b32 needs (0 when it does not split K). */
size_t mxd_gemm_gate_up_q8b32_workspace_size(int n_rows, int F, int K);

/* H[b] = act(Wg · X[b]) ⊙ (Wu · X[b]) for int8 block-32 Wg, Wu [F][K]; H fp32
 * [n_rows][F]. Counterpart of gemm_gate_up_silu (KL/kernels.metal:445-510). */
int mxd_gemm_gate_up_q8b32(const int8_t* Wg, const uint16_t* sg, const int8_t* Wu, const uint16_t* su,
                           const uint16_t* X, float* H, int n_rows, int F, int K, int act, void* workspace,
                           size_t ws_bytes, mxd_stream_t stream);

/* Workspace bytes mxd_gemm_f16 needs (0 when it does not split K). */
size_t mxd_gemm_f16_workspace_size(int n_rows, int M, int K);

/* Y[b] (op)= W · X[b] for fp16 W [M][K] and the n_rows rows of X [n_rows][K]
 * (x_dtype MXD_F16, or MXD_F32 rounded to nearest-even fp16 as it is loaded);
 * Y fp32 [n_rows][M]; epilogue MXD_EPI_STORE or MXD_EPI_ADD; fp32
 * accumulation. From 16 rows on (and K % 128 == 0) this runs on the matrix
 * cores; below, one matvec per row. Replaces gemm_f16 / gemm_f16_add
 * (KL/kernels.metal:376-441; host gemm KL/main.swift:397-410), the prefill
 * products; fp32 X folds the f32_to_f16 cast before them (KL/main.swift:448-454). */
int mxd_gemm_f16(const uint16_t* W, const void* X, int x_dtype, float* Y, int n_rows, int M, int K,
                 int epilogue, void* workspace, size_t ws_bytes, mxd_stream_t stream);

/* Workspace bytes mxd_gemm_gate_up_f16 needs (0 when it does not split K). */
size_t mxd_gemm_gate_up_f16_workspace_size(int n_rows, int F, int K);

/* H[b] = act(Wg · X[b]) ⊙ (Wu · X[b]) for fp16 Wg, Wu [F][K]; H fp32
 * [n_rows][F]. Replaces gemm_gate_up_silu (KL/kernels.metal:445-510; host
 * gemmGateUp KL/main.swift:412-446), with GeGLU as well. */
int mxd_gemm_gate_up_f16(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* X, float* H, int n_rows, int F,
                         int K, int act, void* workspace, size_t ws_bytes, mxd_stream_t stream);

/* ---- decode engine ---------------------------------------------------------- */

/* Model shape. Replaces the reference's Config read from the weight file's JSON
 * header (KL/main.swift:75-110). Weights fp16, norm weights fp32. head_dim 64
 * (Llama-3.2-1B), 128 or 256 (Gemma-2B). */
typedef struct mxd_model_config {
    int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab;
    float rms_eps, rope_theta;
    int act;                  /* MXD_ACT_GELU_TANH (Gemma GeGLU) or MXD_ACT_SILU */
    int norm_plus_one;        /* RMSNorm weight (1 + w) (Gemma) instead of w     */
    int embed_scale_sqrt_dim; /* x = E[tok] * sqrt(dim) (KG/main.swift:397)      */
    int untied_lm_head;       /* logits from a separate "lm_head" tensor
                                 (KL/main.swift:306) instead of the embedding
                                 (tied, KG/main.swift:379-380)                    */
    /* Llama-3 RoPE frequency scaling (rope_scaling rope_type "llama3",
     * KL/main.swift:96-107), applied on the host in double when rope_factor > 0 */
    float rope_factor, rope_low_freq_factor, rope_high_freq_factor;
    int rope_original_max_positions;
} mxd_model_config;

/* Gemma-4 per-layer facts, as the reference's converter resolves them into
 * the weight file's "engine" header (KG/convert_weights.py engine_config;
 * read at KG/main.swift:75-101). */
typedef struct mxd_gemma4_layer {
    int head_dim;     /* 64, 128, 256 (E2B sliding) or 512 (E2B full)              */
    int ffn_dim;      /* doubled on KV-shared layers                               */
    int sliding;      /* 1: attends to the last `window` keys                      */
    int kv_layer;     /* the layer whose K/V cache it reads (itself, or shared)     */
    int rope_pairs;   /* rotated pairs (hd/2 default RoPE; fewer: proportional)    */
    float rope_theta;
    float layer_scalar;
} mxd_gemma4_layer;

/* Gemma-4 text model (KG/main.swift:80-101): tied embedding scaled by
 * sqrt(dim), per-layer embeddings of ple_dim per layer, RMSNorm weights
 * multiplied as stored (w, not 1 + w), attention scale 1 (q/k norms), GeGLU,
 * final logit softcap (applied where logits are read, not before argmax). */
typedef struct mxd_gemma4_config {
    int n_layers, dim, n_heads, n_kv_heads, vocab, ple_dim, ple_vocab, window;
    float rms_eps, softcap;
    const mxd_gemma4_layer* layers; /* n_layers entries, copied at create */
} mxd_gemma4_config;

typedef struct mxd_engine mxd_engine;

/* Allocates weights (one arena, tensors 256-byte aligned as in the reference's
 * flat weight file, KL/convert_weights.py:71-89), activations, a token buffer of
 * max_ctx + 1 ids and fp16 KV caches; owns one HIP stream. Replaces Engine.init
 * (KL/main.swift:168-215). Weights start uninitialised. */
int mxd_engine_create(const mxd_model_config* cfg, int max_ctx, mxd_engine** out);
/* The Gemma-4 engine (KG/main.swift:148-457) behind the same handle: every
 * mxd_engine_* call below serves it. Tensors (KG/convert_weights.py): "embed",
 * "ple_embed" [ple_vocab][n_layers*ple_dim], "ple_proj" [n_layers*ple_dim][dim],
 * "ple_norm", "final_norm", and per layer "l<i>.attn_norm", "l<i>.wqkv" (q|k|v
 * rows; q only on a layer with kv_layer != i), "l<i>.q_norm", "l<i>.k_norm"
 * (own K/V only), "l<i>.wo", "l<i>.post_attn_norm", "l<i>.ffn_norm",
 * "l<i>.wgate", "l<i>.wup", "l<i>.wdown", "l<i>.post_ffn_norm",
 * "l<i>.ple_gate", "l<i>.ple_out", "l<i>.post_ple_norm". K/V caches exist for
 * the layers that own them. mxd_engine_get_logits returns softcapped logits
 * (--dump-logits, KG/main.swift:657-662). */
int mxd_engine_create_gemma4(const mxd_gemma4_config* cfg, int max_ctx, mxd_engine** out);
/* (Its prefill runs chunks of up to 256 rows through the matrix-core
 * * products as encodePrefillChunk does, KG/main.swift:486-520: activations
 * rounded to fp16 before each product, the per-layer inputs' gate through
 * mxd_ple_gate_act; ENG_NO_GEMM = 1 steps the decode path instead.) */
int mxd_engine_destroy(mxd_engine* e);
/* Weight tensors by index / name: "embed", "final_norm", "l<i>.attn_norm",
 * "l<i>.wqkv" (rows q|k|v), "l<i>.wo", "l<i>.ffn_norm", "l<i>.wgate",
 * "l<i>.wup", "l<i>.wdown", and "lm_head" when untied (names of
 * KL/convert_weights.py:56-69). */
int mxd_engine_num_tensors(const mxd_engine* e);
int mxd_engine_tensor(const mxd_engine* e, int index, const char** name, void** dev_ptr, size_t* bytes,
                      int* dtype);
/* Index of a named tensor, or a negative error code. */
int mxd_engine_find_tensor(const mxd_engine* e, const char* name);
/* Copies one tensor's bytes from host memory (the weight-file loader's path),
 * or back to host memory. Both synchronise the engine stream. */
int mxd_engine_upload(mxd_engine* e, int index, const void* host, size_t bytes);
int mxd_engine_download(mxd_engine* e, int index, void* host, size_t bytes);
/* Fills every weight with mxd_fill_normal(seed, tensor id), ids: embed 1,
 * final_norm 2, lm_head 3, layer l: 1000 + 16 l + {attn_norm 0, wqkv 1, wo 2,
 * ffn_norm 3, wgate 4, wup 5, wdown 6}. Gemma-4 adds ple_embed 4, ple_proj 5,
 * ple_norm 6 and per layer {q_norm 7, k_norm 8, post_attn_norm 9,
 * post_ffn_norm 10, ple_gate 11, ple_out 12, post_ple_norm 13}; its norm
 * weights are 1 + the generated value (fp32 sum), as they multiply unshifted.
 * Synchronises. */
int mxd_engine_init_random(mxd_engine* e, uint64_t seed, float stddev);
/* Refills one tensor with mxd_fill_normal(seed, its tensor id, stddev), e.g.
 * the embedding at its own scale. Synchronises. Like init_random, it stands in
 * for the converted checkpoint (KL/convert_weights.py:71-89). */
int mxd_engine_fill_tensor(mxd_engine* e, int index, uint64_t seed, float stddev);
size_t mxd_engine_weight_bytes(const mxd_engine* e);

/* tokens[start .. start+n) from / to host memory (Engine.setTokens / token(at:),
 * KL/main.swift:383-390). Both synchronise the engine stream. */
int mxd_engine_set_tokens(mxd_engine* e, const int32_t* ids, int start, int n);
int mxd_engine_get_tokens(mxd_engine* e, int32_t* ids, int start, int n);
/* The fp32 logits of the last sampled step (--dump-logits, KL/main.swift:572-575). */
int mxd_engine_get_logits(mxd_engine* e, float* host);

/* One decode step at pos: reads tokens[pos], appends K/V at pos and, with
 * sample, writes argmax to tokens[pos + 1]. Asynchronous. Replaces
 * encodeDecode (KL/main.swift:321-347). */
int mxd_engine_step(mxd_engine* e, int pos, int sample);
/* Positions 0..n-1 of tokens[], sampling tokens[n] (prefill(n:useGemm:),
 * KL/main.swift:357-372). From n = 2 the prompt runs in chunks of up to 256
 * rows through mxd_gemm_f16 / mxd_gemm_gate_up_f16, mxd_attention_prefill and
 * row-batched norm / RoPE / casts, with activations rounded to fp16 before each
 * product as the reference's chunk does (encodePrefillChunk,
 * KL/main.swift:412-446); the last row takes the decode path's LM head. With
 * the ENG_NO_GEMM tunable set to 1 (the reference's --no-gemm) it steps the
 * decode path token by token (KL/main.swift:367-368). Asynchronous. */
int mxd_engine_prefill(mxd_engine* e, int n);
/* count greedy steps from pos (tokens[pos] must be set) with no host round trip:
 * one captured graph replayed per step, the position kept on the device.
 * Replaces Engine.decode(from:count:) (KL/main.swift:376-381). Asynchronous. */
int mxd_engine_decode(mxd_engine* e, int pos, int count);
/* Waits for the engine stream (waitUntilCompleted, KL/main.swift:379). */
int mxd_engine_sync(mxd_engine* e);
/* Waits until the step at pos queued by mxd_engine_decode has finished, without
 * waiting for the steps queued after it, and returns the token it sampled
 * (tokens[pos + 1]). Each decode step writes its token to pinned host memory
 * and records an event in a ring of 16 steps, so a caller keeps several steps
 * in flight and waits on the oldest: the per-command-buffer wait of
 * decodeStreaming (KL/main.swift:477-491). Valid for a pos decoded since the
 * last prefill / step at that position. */
int mxd_engine_wait_token(mxd_engine* e, int pos, int32_t* token);

#ifdef __cplusplus
}
#endif

#endif /* MXDECODE_H */
