// Library-internal launchers shared between translation units (not part of
// the C ABI). The *_dev variants read the step position from device memory
// when pos_dev is not null, so a captured decode step replays at a moving
// position without host involvement.
#pragma once

#include "common.hpp"

namespace mxd {

// With step_counter, the kernel also advances *step_counter by one (the decode
// step count the fused attention block derives its tags from).
int embed_dev(const uint16_t* E, const int32_t* tokens, int pos, const int32_t* pos_dev, int rows, float* x, int D,
              float scale, int vocab, hipStream_t s, int32_t* step_counter = nullptr);

// The fused attention half of a decode layer (attn_block.hip): x +=
// Wo . attention(RoPE(q), K, V) with [q|k|v] = Wqkv . rmsnorm(x), the new k, v
// appended at pos (or *pos_dev), in one launch. step_dev: a counter advanced
// once per decode step; layer < 64 tells the layers of a step apart.
size_t attn_block_workspace_size(int n_heads, int n_kv, int hd, int max_ctx);
int attn_block(const uint16_t* wqkv, const uint16_t* wo, float* x, const float* norm_w, float eps, int plus_one,
               uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads, int n_kv, int hd, int dim,
               int max_ctx, int pos, const int32_t* pos_dev, float scale, const int32_t* step_dev, int layer,
               void* workspace, size_t ws_bytes, hipStream_t s);
int* attn_block_err(void* workspace, int n_heads, int n_kv, int hd, int max_ctx);

int rope_kv_dev(float* qkv, uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads, int n_kv, int hd,
                int max_ctx, int pos0, int rows, const int32_t* pos_dev, hipStream_t s);

// tokens[pos + 1] (or tokens[out_idx] without pos_dev) = argmax; with advance,
// *pos_dev += 1 afterwards. With host_tokens (device-visible pinned host
// memory) the token is also written to host_tokens at the same index.
int argmax_dev(const float* logits, int32_t* tokens, int N, int out_idx, int32_t* pos_dev, bool advance,
               void* workspace, hipStream_t s, int32_t* host_tokens = nullptr);

// mxd_fill_normal with every fp32 value then shifted by `shift` (fp32 add;
// shift != 0 needs MXD_F32).
int fill_normal_dev(void* dst, int dtype, uint64_t n, uint64_t seed, uint64_t tensor_id, float stddev, float shift,
                    hipStream_t s);

// fp16 (MXD_W_F16) or int8 block-32 (MXD_W_Q8B32) matvec whose fp32 x is
// rounded to fp16 as it is loaded.
int matvec_xr16(int w_format, const void* W, const uint16_t* scales, const float* x, float* y, int M, int K,
                int epilogue, hipStream_t s);

// Prefill with fp16 activation rows between ops (the engines' prefill rounds
// the attention and hidden rows to fp16 before the products that read them;
// writing them as fp16 lets those products stage fp16 rows):
// mxd_attention_prefill_window with fp16 output rows (out_stride halfs apart),
// and mxd_gemm_gate_up_f16 with fp16 H.
int attention_prefill_h16(const float* q, int q_stride, const uint16_t* kcache, const uint16_t* vcache, uint16_t* out,
                          int out_stride, int n_heads, int n_kv_heads, int head_dim, int max_ctx, int pos0, int rows,
                          int window, float scale, hipStream_t stream);
int gemm_gate_up_f16_h16(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* X, uint16_t* H, int n_rows, int F,
                         int K, int act, void* workspace, size_t ws_bytes, hipStream_t stream);
// Whether an fp16 product of n_rows rows and depth K runs on the matrix cores
// (gemm_gate_up_f16_h16 needs it; below, the products run one matvec per row).
bool gemm_on_matrix_cores(int n_rows, int K);

}  // namespace mxd
