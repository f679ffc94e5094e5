// Device building blocks of the single-token matvecs, shared by the matvec
// kernels (gemv.hip) and the fused decode attention block (attn_block.hip):
// the argument block, activation fragments, the 16-byte partial dot products,
// the RoPE row pairing and the fused RMSNorm scale.
#pragma once

#include "internal.hpp"

namespace {

enum { WF_F32 = 2 };

template <int WF> struct WT;
template <> struct WT<MXD_W_F16> { static constexpr int EPL = 8; };    // 8 halfs in 16 B
template <> struct WT<MXD_W_Q8B32> { static constexpr int EPL = 16; }; // 16 int8 in 16 B
template <> struct WT<WF_F32> { static constexpr int EPL = 4; };       // 4 floats in 16 B

struct GemvArgs {
    const void* W[2];
    const uint16_t* S[2];
    const void* x;
    float* y;
    const float* aux;
    int M, K;
    // Optional fused RMSNorm of x (fp32 x): x_k * rsqrt(mean(x^2) + eps) * w_k
    // (or * (1 + w_k)), computed by every workgroup in a prologue.
    const float* nw = nullptr;
    float eps = 0.0f;
    int plus_one = 0;
    // RoPE + KV-append epilogue of the fused q|k|v projection (EPI_ROPE_KV).
    const float* inv_freq = nullptr;
    uint16_t* kcache = nullptr;
    uint16_t* vcache = nullptr;
    const int32_t* pos_dev = nullptr;
    int pos = 0, n_heads = 0, n_kv = 0, hd = 0, max_ctx = 0;
    // x as the log-sum-exp merge of single-query attention partials
    // (mxd_attention_split: O [splits][n_heads][hd], (max, sum) [splits][n_heads][2],
    // log2 domain); the active splits follow from the key count n_keys, or
    // *pos_dev + 1, as in the producer.
    const float* mpo = nullptr;
    const float* mpml = nullptr;
    int msplits = 0, n_keys = 0;
    int mwindow = 0;  // the producer's sliding window (0: all keys)
    // fp32 x rounded to nearest-even fp16 on load (the batched products'
    // fp32-activation mode, below their matrix-core threshold)
    int xr16 = 0;
    // Residual prologue (a sandwich norm's residual add folded into the next
    // product): the product's x is x' = (x + rsrc * rsqrt(mean(rsrc^2) + eps)
    // * rw) * rpost, formed by every workgroup in dynamic LDS (K floats) and
    // written to rout by workgroup 0 (rout != x: the other workgroups still
    // read x).
    const float* rsrc = nullptr;
    const float* rw = nullptr;
    float rpost = 1.0f;
    float* rout = nullptr;
};

constexpr int MERGE_MAX_SPLITS = 8;

// Splits of a key count that hold a partial (one per 32-key block, at most
// msplits, at least one: an empty context leaves one zero partial).
__device__ __forceinline__ int merge_active(const GemvArgs& a) {
    int n = a.pos_dev ? a.pos_dev[0] + 1 : a.n_keys;
    n = max(0, min(n, a.max_ctx));
    const int lo = a.mwindow > 0 ? max(0, n - a.mwindow) : 0;  // blocks before the window hold none
    return max(1, min(a.msplits, (n + 31) / 32 - lo / 32));
}

// Internal epilogue: rows are rotated in (i, i + hd/2) pairs and q goes back
// to y while k and v are appended to the tiled caches.
constexpr int EPI_ROPE_KV = 16;

// EPL activation values starting at column c.
template <typename XT, int EPL> struct XFrag;

template <int EPL> struct XFrag<float, EPL> {
    float v[EPL];
    __device__ __forceinline__ void load(const void* x, int c, int round16 = 0) {
        const float* p = static_cast<const float*>(x) + c;
#pragma unroll
        for (int i = 0; i < EPL / 4; ++i) {
            const f4_t t = *reinterpret_cast<const f4_t*>(p + 4 * i);
            v[4 * i + 0] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
        if (round16) {
#pragma unroll
            for (int i = 0; i < EPL; ++i) v[i] = (float)(_Float16)v[i];
        }
    }
    // x_k * scale * w_k (or * (1 + w_k)): the fused RMSNorm, same operation
    // order as the standalone kernel.
    __device__ __forceinline__ void load_norm(const void* x, const float* w, int c, float scale, int plus_one) {
        load(x, c);
#pragma unroll
        for (int i = 0; i < EPL / 4; ++i) {
            const f4_t t = *reinterpret_cast<const f4_t*>(w + c + 4 * i);
            const float wv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) v[4 * i + j] = v[4 * i + j] * scale * (plus_one ? 1.0f + wv[j] : wv[j]);
        }
    }
    // x[c .. c + EPL) merged from the attention partials: the EPL values lie in
    // one head h (hd % EPL == 0); x = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
    // Every split's loads go out before any math.
    __device__ __forceinline__ void load_merge(const GemvArgs& a, int c) {
        const int h = c / a.hd, na = merge_active(a);
        const size_t ostride = (size_t)a.n_heads * a.hd, mlstride = (size_t)a.n_heads * 2;
        float m[MERGE_MAX_SPLITS], l[MERGE_MAX_SPLITS];
        f4_t o[MERGE_MAX_SPLITS][EPL / 4];
#pragma unroll
        for (int sp = 0; sp < MERGE_MAX_SPLITS; ++sp) {
            if (sp >= na) break;
            m[sp] = a.mpml[sp * mlstride + 2 * h];
            l[sp] = a.mpml[sp * mlstride + 2 * h + 1];
#pragma unroll
            for (int i = 0; i < EPL / 4; ++i) o[sp][i] = *reinterpret_cast<const f4_t*>(a.mpo + sp * ostride + c + 4 * i);
        }
        float M = m[0];
#pragma unroll
        for (int sp = 1; sp < MERGE_MAX_SPLITS; ++sp)
            if (sp < na) M = fmaxf(M, m[sp]);
        float L = 0.0f;
        f4_t acc[EPL / 4];
#pragma unroll
        for (int i = 0; i < EPL / 4; ++i) acc[i] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sp = 0; sp < MERGE_MAX_SPLITS; ++sp) {
            if (sp >= na) break;
            const float f = __builtin_amdgcn_exp2f(m[sp] - M);
            L += f * l[sp];
#pragma unroll
            for (int i = 0; i < EPL / 4; ++i) acc[i] += f * o[sp][i];
        }
        const float inv = 1.0f / L;
#pragma unroll
        for (int i = 0; i < EPL / 4; ++i) {
            v[4 * i + 0] = acc[i].x * inv;
            v[4 * i + 1] = acc[i].y * inv;
            v[4 * i + 2] = acc[i].z * inv;
            v[4 * i + 3] = acc[i].w * inv;
        }
    }
};

template <int EPL> struct XFrag<_Float16, EPL> {
    h2_t v[EPL / 2];
    __device__ __forceinline__ void load_norm(const void*, const float*, int, float, int) {}  // host rejects
    __device__ __forceinline__ void load_merge(const GemvArgs&, int) {}                      // host rejects
    __device__ __forceinline__ void load(const void* x, int c, int = 0) {
        const _Float16* p = static_cast<const _Float16*>(x) + c;
#pragma unroll
        for (int i = 0; i < EPL / 8; ++i) {
            const u4_t t = *reinterpret_cast<const u4_t*>(p + 8 * i);
            v[4 * i + 0] = mxd::as_h2(t.x);
            v[4 * i + 1] = mxd::as_h2(t.y);
            v[4 * i + 2] = mxd::as_h2(t.z);
            v[4 * i + 3] = mxd::as_h2(t.w);
        }
    }
};

// ---- partial dot products: acc + w . x over one lane's 16 bytes -----------

__device__ __forceinline__ float dot16(u4_t w, const XFrag<float, 8>& x, float acc) {  // fp16 W
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h2_t h = mxd::as_h2(w[j]);
        acc = fmaf((float)h.x, x.v[2 * j], acc);
        acc = fmaf((float)h.y, x.v[2 * j + 1], acc);
    }
    return acc;
}

__device__ __forceinline__ float dot16(u4_t w, const XFrag<_Float16, 8>& x, float acc) {  // fp16 W
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_fdot2(mxd::as_h2(w[j]), x.v[j], acc, false);
    return acc;
}

__device__ __forceinline__ float dot16(u4_t w, const XFrag<float, 4>& x, float acc) {  // fp32 W
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(__uint_as_float(w[j]), x.v[j], acc);
    return acc;
}

// int8 weights: the sum over half a quantisation block (16 weights), unscaled.
__device__ __forceinline__ float dot16q(u4_t w, const XFrag<_Float16, 16>& x) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h2_t lo, hi;
        mxd::i8x4_to_h2x2(w[j], lo, hi);
        s = __builtin_amdgcn_fdot2(lo, x.v[2 * j], s, false);
        s = __builtin_amdgcn_fdot2(hi, x.v[2 * j + 1], s, false);
    }
    return s;
}

__device__ __forceinline__ float dot16q(u4_t w, const XFrag<float, 16>& x) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h2_t lo, hi;
        mxd::i8x4_to_h2x2(w[j], lo, hi);
        s = fmaf((float)lo.x, x.v[4 * j + 0], s);
        s = fmaf((float)lo.y, x.v[4 * j + 1], s);
        s = fmaf((float)hi.x, x.v[4 * j + 2], s);
        s = fmaf((float)hi.y, x.v[4 * j + 3], s);
    }
    return s;
}

template <int WF>
__device__ __forceinline__ size_t welem_bytes() {
    return WF == MXD_W_F16 ? 2 : WF == MXD_W_Q8B32 ? 1 : 4;
}

// Weights are read exactly once per call: nontemporal loads keep them from
// displacing the activations and partial sums that are reused from cache.
template <int WF>
__device__ __forceinline__ u4_t ld_stream(const unsigned char* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p));
}

// For EPI_ROPE_KV the workgroup rows are "virtual": consecutive pairs map to
// the rotation partners (i, i + hd/2) of one q or k head, so the epilogue holds
// both; the v rows (after all q and k rows) map to themselves.
__device__ __forceinline__ int rope_row(int v, const GemvArgs& a) {
    const int half = a.hd >> 1;
    if (v >= (a.n_heads + a.n_kv) * a.hd) return v;
    const int p = v >> 1, head = p / half, i = p - head * half;
    return head * a.hd + i + (v & 1) * half;
}

// rsqrt(mean(x^2) + eps) of the fp32 vector x[0..K), reduced by the whole
// workgroup (K % 4 == 0).
template <int NW>
__device__ __forceinline__ float block_rms_scale(const float* x, int K, float eps) {
    __shared__ float nred[NW];
    float ss = 0.0f;
    for (int k = threadIdx.x * 4; k < K; k += NW * 64 * 4) {
        const f4_t t = *reinterpret_cast<const f4_t*>(x + k);
        ss = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, ss))));
    }
    ss = mxd::wave_sum(ss);
    if ((threadIdx.x & 63) == 0) nred[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = nred[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) tot += nred[w];
    return rsqrtf(tot / (float)K + eps);
}

// The residual prologue (GemvArgs::rsrc): forms x' in dynamic LDS and points
// a.x at it. Every thread of the workgroup calls it before any x load; the
// kernels issue their first weight loads before it, so the prologue's round
// trip overlaps them. For K up to 4096 x (NW / 4) it loads src, x and w in one
// pass and keeps them in registers through the rms reduction (the sum of
// squares in the same per-thread order as block_rms_scale).
template <int NW>
__device__ __forceinline__ void residual_prologue(GemvArgs& a) {
    if (!a.rsrc) return;
    extern __shared__ __attribute__((aligned(16))) float gemv_dyn_x[];
    constexpr int T = NW * 64;
    constexpr int IT = 4096 / (T * 4) > 0 ? 4096 / (T * 4) : 1;  // f4 per thread held in registers
    const int K = a.K;
    const float* x = static_cast<const float*>(a.x);
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && a.rout != nullptr;
    auto finish = [&](int k, const f4_t& xv, const f4_t& sv, const f4_t& wv, float scale) {
        f4_t v;
        v.x = (xv.x + sv.x * scale * wv.x) * a.rpost;
        v.y = (xv.y + sv.y * scale * wv.y) * a.rpost;
        v.z = (xv.z + sv.z * scale * wv.z) * a.rpost;
        v.w = (xv.w + sv.w * scale * wv.w) * a.rpost;
        *reinterpret_cast<f4_t*>(gemv_dyn_x + k) = v;
        if (writer) *reinterpret_cast<f4_t*>(a.rout + k) = v;
    };
    if (K <= IT * T * 4) {
        __shared__ float nred[NW];
        f4_t xv[IT], sv[IT], wv[IT];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int k = (threadIdx.x + i * T) * 4;
            if (k < K) {
                sv[i] = *reinterpret_cast<const f4_t*>(a.rsrc + k);
                xv[i] = *reinterpret_cast<const f4_t*>(x + k);
                wv[i] = *reinterpret_cast<const f4_t*>(a.rw + k);
            }
        }
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int k = (threadIdx.x + i * T) * 4;
            if (k < K) {
                const f4_t t = sv[i];
                ss = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, ss))));
            }
        }
        ss = mxd::wave_sum(ss);
        if ((threadIdx.x & 63) == 0) nred[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = nred[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) tot += nred[w];
        const float scale = rsqrtf(tot / (float)K + a.eps);
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int k = (threadIdx.x + i * T) * 4;
            if (k < K) finish(k, xv[i], sv[i], wv[i], scale);
        }
    } else {
        const float scale = block_rms_scale<NW>(a.rsrc, K, a.eps);
        for (int k = threadIdx.x * 4; k < K; k += T * 4)
            finish(k, *reinterpret_cast<const f4_t*>(x + k), *reinterpret_cast<const f4_t*>(a.rsrc + k),
                   *reinterpret_cast<const f4_t*>(a.rw + k), scale);
    }
    __syncthreads();
    a.x = gemv_dyn_x;
}

}  // namespace
