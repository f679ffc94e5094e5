// RMSNorm, embedding lookup, fp32->fp16 cast, and RoPE with KV-cache append.
// These move kilobytes per decode step; they are latency-bound, so each is a
// single small launch with no host synchronisation.
#include <type_traits>

#include "internal.hpp"

namespace {

constexpr int NORM_THREADS = 256;

// Sum over a 256-thread workgroup; every thread receives the total.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = mxd::wave_sum(v);
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = scratch[0];
#pragma unroll
    for (int w = 1; w < NORM_THREADS / 64; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

// y = x * rsqrt(mean(x^2) + eps) * (1 + w | w), one workgroup per row
// (KL/kernels.metal:71-96).
// Rows of up to NORM_CACHE * 4 * NORM_THREADS floats (D % 4 == 0) are read once
// with 16-byte loads, all in flight together, and kept in registers for the
// second pass; other rows take the plain two-pass loop.
constexpr int NORM_CACHE = 8;

template <typename YT, bool PLUS_ONE>
__global__ void __launch_bounds__(NORM_THREADS)
rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, YT* __restrict__ y, int D, float eps) {
    __shared__ float scratch[NORM_THREADS / 64];
    const float* xr = x + (size_t)blockIdx.x * D;
    YT* yr = y + (size_t)blockIdx.x * D;
    if (D % 4 == 0 && D <= NORM_CACHE * 4 * NORM_THREADS) {
        f4_t v[NORM_CACHE];
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < NORM_CACHE; ++u) {
            const int i = (threadIdx.x + u * NORM_THREADS) * 4;
            v[u] = i < D ? *reinterpret_cast<const f4_t*>(xr + i) : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < NORM_CACHE; ++u)
            ss = fmaf(v[u].x, v[u].x, fmaf(v[u].y, v[u].y, fmaf(v[u].z, v[u].z, fmaf(v[u].w, v[u].w, ss))));
        ss = block_sum(ss, scratch);
        const float scale = rsqrtf(ss / (float)D + eps);
#pragma unroll
        for (int u = 0; u < NORM_CACHE; ++u) {
            const int i = (threadIdx.x + u * NORM_THREADS) * 4;
            if (i < D) {
                const f4_t wv = *reinterpret_cast<const f4_t*>(w + i);
                const float xs[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                const float ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) yr[i + e] = (YT)(xs[e] * scale * (PLUS_ONE ? 1.0f + ws[e] : ws[e]));
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, scratch);
    const float scale = rsqrtf(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) {
        const float wi = PLUS_ONE ? 1.0f + w[i] : w[i];
        yr[i] = (YT)(xr[i] * scale * wi);
    }
}

// The sum of the K-split partials at element e (split stride `stride`),
// added in split order from zero: the same order as the products' own
// reduction, so the result is bit-identical to the summed output. With NS > 0
// (the split count known at compile time) every load is issued before the
// first add, one round trip in all; NS == 0 takes the runtime count n.
template <int NS, typename T>
__device__ __forceinline__ T split_sum(const float* __restrict__ part, int n, size_t stride, size_t e) {
    T t{};
    if constexpr (NS == 0) {
        for (int sp = 0; sp < n; ++sp) t += *reinterpret_cast<const T*>(part + sp * stride + e);
    } else {
        T v[NS];
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) v[sp] = *reinterpret_cast<const T*>(part + sp * stride + e);
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) t += v[sp];
    }
    return t;
}

// Calls f(std::integral_constant<int, NS>) with NS = n for 1 <= n <= 8 and
// NS = 0 (a runtime count) otherwise.
template <typename F>
int with_splits(int n, F&& f) {
    switch (n) {
        case 1: return f(std::integral_constant<int, 1>{});
        case 2: return f(std::integral_constant<int, 2>{});
        case 3: return f(std::integral_constant<int, 3>{});
        case 4: return f(std::integral_constant<int, 4>{});
        case 5: return f(std::integral_constant<int, 5>{});
        case 6: return f(std::integral_constant<int, 6>{});
        case 7: return f(std::integral_constant<int, 7>{});
        case 8: return f(std::integral_constant<int, 8>{});
        default: return f(std::integral_constant<int, 0>{});
    }
}

// x[r] += sum of the K-split partials of a product's row r (the residual add
// the product would have done), then y[r] = rmsnorm(x[r]) as rmsnorm_kernel
// computes it (same loads per thread and the same reduction order), one
// workgroup per row. All of a thread's loads go out before its first add.
template <typename YT, bool PLUS_ONE, int NS, int NC>
__global__ void __launch_bounds__(NORM_THREADS)
rmsnorm_residual_sum_kernel(float* __restrict__ x, const float* __restrict__ part, int n_splits, size_t stride,
                            const float* __restrict__ w, YT* __restrict__ y, int D, float eps) {
    __shared__ float scratch[NORM_THREADS / 64];
    const size_t r0 = (size_t)blockIdx.x * D;
    float* xr = x + r0;
    YT* yr = y + r0;
    // NC 16-byte groups per thread (NC * 4 * NORM_THREADS >= D): rmsnorm_kernel's
    // cached loop, whose groups past D add exact zeros to the sum of squares.
    // Loads past D read the row's first group instead (no masked blocks, so
    // every load is issued before the first wait) and are then zeroed.
    if (NC > 0 && D % 4 == 0 && D <= NC * 4 * NORM_THREADS) {
        constexpr int NU = NC > 0 ? NC : 1;
        constexpr int NP = NS > 0 ? NS : 1;
        f4_t v[NU];
        f4_t pv[NU][NP];
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int i = (threadIdx.x + u * NORM_THREADS) * 4;
            const int ic = i < D ? i : 0;
            v[u] = *reinterpret_cast<const f4_t*>(xr + ic);
            if constexpr (NS > 0) {
#pragma unroll
                for (int sp = 0; sp < NS; ++sp) pv[u][sp] = *reinterpret_cast<const f4_t*>(part + sp * stride + r0 + ic);
            } else {
                pv[u][0] = split_sum<0, f4_t>(part, n_splits, stride, r0 + ic);
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int i = (threadIdx.x + u * NORM_THREADS) * 4;
            f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int sp = 0; sp < NP; ++sp) acc += pv[u][sp];
            const f4_t t = v[u] + acc;
            v[u] = i < D ? t : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
            if (i < D) *reinterpret_cast<f4_t*>(xr + i) = t;
        }
#pragma unroll
        for (int u = 0; u < NU; ++u)
            ss = fmaf(v[u].x, v[u].x, fmaf(v[u].y, v[u].y, fmaf(v[u].z, v[u].z, fmaf(v[u].w, v[u].w, ss))));
        ss = block_sum(ss, scratch);
        const float scale = rsqrtf(ss / (float)D + eps);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int i = (threadIdx.x + u * NORM_THREADS) * 4;
            if (i < D) {
                const f4_t wv = *reinterpret_cast<const f4_t*>(w + i);
                const float xs[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                const float ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) yr[i + e] = (YT)(xs[e] * scale * (PLUS_ONE ? 1.0f + ws[e] : ws[e]));
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) {
        const float t = xr[i] + split_sum<NS, float>(part, n_splits, stride, r0 + i);
        xr[i] = t;
        ss = fmaf(t, t, ss);
    }
    ss = block_sum(ss, scratch);
    const float scale = rsqrtf(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) {
        const float wi = PLUS_ONE ? 1.0f + w[i] : w[i];
        yr[i] = (YT)(xr[i] * scale * wi);
    }
}

// x[r][i] = float(E[tokens[pos + r]][i]) * scale; ids outside [0, vocab) give
// a zero row instead of an out-of-bounds read.
// With pos_dev set, the position is read on the device (a replayed step).
__global__ void __launch_bounds__(256) embed_kernel(const uint16_t* __restrict__ E, const int32_t* __restrict__ tokens,
                                                    int pos, const int32_t* __restrict__ pos_dev, float* __restrict__ x,
                                                    int D, float scale, int vocab, int32_t* step_counter) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (step_counter && i == 0 && r == 0) step_counter[0] += 1;
    if (i >= D) return;
    if (pos_dev) pos = pos_dev[0];
    const int tok = tokens[pos + r];
    x[(size_t)r * D + i] = (tok >= 0 && tok < vocab) ? mxd::h2f(E[(size_t)tok * D + i]) * scale : 0.0f;
}

__global__ void __launch_bounds__(256) f32_to_f16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                         size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = mxd::f2h_bits(src[i]);
}

// One thread per rotation pair (i, i + hd/2) per head per row; heads run over
// the q heads, then the kv heads (KL/kernels.metal:182-224). K and V go to
// the tiled caches.
__global__ void __launch_bounds__(256)
rope_kv_kernel(float* __restrict__ qkv, uint16_t* __restrict__ kcache, uint16_t* __restrict__ vcache,
               const float* __restrict__ inv_freq, int n_heads, int n_kv, int hd, int max_ctx, int pos0,
               const int32_t* __restrict__ pos_dev) {
    const int half_d = hd >> 1;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index over heads
    const int t = blockIdx.y;                              // row
    const int h = i / half_d, p = i - h * half_d;
    if (h >= n_heads + n_kv) return;
    if (pos_dev) pos0 = pos_dev[0];
    if (pos0 < 0 || pos0 + t >= max_ctx) return;  // a device position past the cache writes nothing
    const int row_len = (n_heads + 2 * n_kv) * hd;
    const int pos = pos0 + t;
    float* row = qkv + (size_t)t * row_len;
    float* v = row + h * hd;
    const float ang = (float)pos * inv_freq[p];
    float s, c;
    sincosf(ang, &s, &c);
    const float a = v[p], b = v[p + half_d];
    const float ra = a * c - b * s;
    const float rb = b * c + a * s;
    if (h < n_heads) {
        v[p] = ra;
        v[p + half_d] = rb;
    } else {
        const int kvh = h - n_heads;
        const size_t tile = ((size_t)kvh * max_ctx + (pos & ~31)) * hd;
        const int k = pos & 31;
        kcache[tile + mxd::k_tile_offset(k, p, hd)] = mxd::f2h_bits(ra);
        kcache[tile + mxd::k_tile_offset(k, p + half_d, hd)] = mxd::f2h_bits(rb);
        const float* vv = row + (n_heads + n_kv + kvh) * hd;
        vcache[tile + mxd::v_tile_offset(k, p)] = mxd::f2h_bits(vv[p]);
        vcache[tile + mxd::v_tile_offset(k, p + half_d)] = mxd::f2h_bits(vv[p + half_d]);
    }
}

// Batched decode over a paged cache: row b of qkv is sequence b's new token,
// at position seq_lens[b] - 1. q and k are rotated in place (as rope_kv does)
// and k, v go to that position's page (slab layouts in common.hpp). A row
// whose position is outside its page-table row, or whose page id is outside
// the pool, is left untouched.
__global__ void __launch_bounds__(256)
rope_kv_paged_kernel(float* __restrict__ qkv, uint16_t* __restrict__ kpool, uint16_t* __restrict__ vpool,
                     const float* __restrict__ inv_freq, int n_heads, int n_kv, int hd,
                     const int32_t* __restrict__ page_table, int max_pages, const int32_t* __restrict__ seq_lens,
                     int n_pages) {
    const int half_d = hd >> 1;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index over heads
    const int b = blockIdx.y;                              // sequence
    const int h = i / half_d, p = i - h * half_d;
    if (h >= n_heads + n_kv) return;
    const int pos = seq_lens[b] - 1;
    if (pos < 0 || pos >= max_pages * mxd::PAGE_KEYS) return;
    const int phys = page_table[(size_t)b * max_pages + (pos >> 4)];
    if (phys < 0 || phys >= n_pages) return;
    float* row = qkv + (size_t)b * (n_heads + 2 * n_kv) * hd;
    float* v = row + h * hd;
    const float ang = (float)pos * inv_freq[p];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float x0 = v[p], x1 = v[p + half_d];
    const float ra = x0 * cs - x1 * sn;
    const float rb = x1 * cs + x0 * sn;
    v[p] = ra;
    v[p + half_d] = rb;
    if (h >= n_heads) {
        const int kvh = h - n_heads, r = pos & (mxd::PAGE_KEYS - 1);
        const size_t slab = ((size_t)phys * n_kv + kvh) * mxd::PAGE_KEYS * hd;
        kpool[slab + mxd::k_page_offset(r, p)] = mxd::f2h_bits(ra);
        kpool[slab + mxd::k_page_offset(r, p + half_d)] = mxd::f2h_bits(rb);
        const float* vv = row + (n_heads + n_kv + kvh) * hd;
        vpool[slab + mxd::v_page_offset(r, p)] = mxd::f2h_bits(vv[p]);
        vpool[slab + mxd::v_page_offset(r, p + half_d)] = mxd::f2h_bits(vv[p + half_d]);
    }
}

// rope_kv_paged_kernel over the K-split partials of the q|k|v product (split
// stride `stride` floats, rows of (n_heads + 2 n_kv) * hd): each value is the
// partials' sum in split order (bit-identical to the summed product), the
// rotated q goes to qkv (the only part of qkv the attention reads) and k, v
// to the pages. A row whose position or page is out of range gets its q
// unrotated, as rope_kv_paged leaves it. A thread's partial loads (its q or k
// pair, and the v pair for a kv head) all go out before the first add.
template <int NS>
__global__ void __launch_bounds__(256)
rope_kv_paged_sum_kernel(const float* __restrict__ part, int n_splits, size_t stride, float* __restrict__ qkv,
                         uint16_t* __restrict__ kpool, uint16_t* __restrict__ vpool,
                         const float* __restrict__ inv_freq, int n_heads, int n_kv, int hd,
                         const int32_t* __restrict__ page_table, int max_pages, const int32_t* __restrict__ seq_lens,
                         int n_pages) {
    const int half_d = hd >> 1;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index over heads
    const int b = blockIdx.y;                              // sequence
    const int h = i / half_d, p = i - h * half_d;
    if (h >= n_heads + n_kv) return;
    const bool kv = h >= n_heads;
    const size_t row = (size_t)b * (n_heads + 2 * n_kv) * hd;
    const size_t e0 = row + (size_t)h * hd + p;
    const size_t v0 = row + (size_t)(h + n_kv) * hd + p;  // the v pair of kv head h - n_heads
    float x0, x1, y0 = 0.0f, y1 = 0.0f;
    if constexpr (NS > 0) {
        // v0 lies inside the row for every head (h + n_kv < n_heads + 2 n_kv), so
        // the v loads need no branch; q heads ignore them
        float a[NS], c[NS], va[NS], vc[NS];
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) {
            a[sp] = part[sp * stride + e0];
            c[sp] = part[sp * stride + e0 + half_d];
            va[sp] = part[sp * stride + v0];
            vc[sp] = part[sp * stride + v0 + half_d];
        }
        x0 = 0.0f, x1 = 0.0f;
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) x0 += a[sp], x1 += c[sp], y0 += va[sp], y1 += vc[sp];
    } else {
        x0 = split_sum<0, float>(part, n_splits, stride, e0);
        x1 = split_sum<0, float>(part, n_splits, stride, e0 + half_d);
        if (kv) {
            y0 = split_sum<0, float>(part, n_splits, stride, v0);
            y1 = split_sum<0, float>(part, n_splits, stride, v0 + half_d);
        }
    }
    const int pos = seq_lens[b] - 1;
    const int phys = pos >= 0 && pos < max_pages * mxd::PAGE_KEYS ? page_table[(size_t)b * max_pages + (pos >> 4)] : -1;
    if (phys < 0 || phys >= n_pages) {
        if (!kv) {
            qkv[e0] = x0;
            qkv[e0 + half_d] = x1;
        }
        return;
    }
    const float ang = (float)pos * inv_freq[p];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float ra = x0 * cs - x1 * sn;
    const float rb = x1 * cs + x0 * sn;
    if (!kv) {
        qkv[e0] = ra;
        qkv[e0 + half_d] = rb;
        return;
    }
    const int kvh = h - n_heads, r = pos & (mxd::PAGE_KEYS - 1);
    const size_t slab = ((size_t)phys * n_kv + kvh) * mxd::PAGE_KEYS * hd;
    kpool[slab + mxd::k_page_offset(r, p)] = mxd::f2h_bits(ra);
    kpool[slab + mxd::k_page_offset(r, p + half_d)] = mxd::f2h_bits(rb);
    vpool[slab + mxd::v_page_offset(r, p)] = mxd::f2h_bits(y0);
    vpool[slab + mxd::v_page_offset(r, p + half_d)] = mxd::f2h_bits(y1);
}

// ---- Gemma-4 operators --------------------------------------------------------

// Sandwich-norm residual update, one workgroup per row (KG/kernels.metal:100-125):
//   x[r][i] = (x[r][i] + src[r][i] * rsqrt(mean(src[r]^2) + eps) * w[i]) * post
// post is the layer scalar after a layer's last residual add, else 1.
__global__ void __launch_bounds__(NORM_THREADS)
rmsnorm_add_kernel(const float* __restrict__ src, const float* __restrict__ w, float* __restrict__ x, int D, float eps,
                   float post) {
    __shared__ float scratch[NORM_THREADS / 64];
    const float* sr = src + (size_t)blockIdx.x * D;
    float* xr = x + (size_t)blockIdx.x * D;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) ss = fmaf(sr[i], sr[i], ss);
    ss = block_sum(ss, scratch);
    const float scale = rsqrtf(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) xr[i] = (xr[i] + sr[i] * scale * w[i]) * post;
}

// Per-layer-embedding combine, one workgroup per (layer slice, row) of P values
// (KG/kernels.metal:127-149):
//   ple[r][l][i] = (rmsnorm(proj[r][l] * proj_scale)[i] * w[i] + ple[r][l][i]) / sqrt(2)
// ple holds the scaled token-identity embedding on entry.
__global__ void __launch_bounds__(NORM_THREADS)
ple_combine_kernel(const float* __restrict__ proj, float* __restrict__ ple, const float* __restrict__ w, int P,
                   int LP, float proj_scale, float eps) {
    __shared__ float scratch[NORM_THREADS / 64];
    const size_t base = (size_t)blockIdx.y * LP + (size_t)blockIdx.x * P;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < P; i += NORM_THREADS) {
        const float v = proj[base + i] * proj_scale;
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, scratch);
    const float scale = rsqrtf(ss / (float)P + eps);
    for (int i = threadIdx.x; i < P; i += NORM_THREADS) {
        const float v = proj[base + i] * proj_scale;
        ple[base + i] = (v * scale * w[i] + ple[base + i]) * 0.70710678118654752f;
    }
}

// Per-head RMSNorm of q and k (weights q_w, k_w) and v (no weight), RoPE on q
// and k over the first rope_pairs rotation pairs (the rest are the identity),
// and the k, v append (KG/kernels.metal:236-304). qkv rows are
// [q n_heads*hd | k n_kv*hd | v n_kv*hd], row t at position pos0 + t (or
// *pos_dev + t); with n_kv == 0 (a KV-shared layer) only q is there. One
// workgroup per (head, row), thread i of hd/2 owns the pair (i, i + hd/2).
__global__ void __launch_bounds__(256)
qk_norm_rope_kernel(float* __restrict__ qkv, uint16_t* __restrict__ kcache, uint16_t* __restrict__ vcache,
                    const float* __restrict__ q_w, const float* __restrict__ k_w, const float* __restrict__ inv_freq,
                    int n_heads, int n_kv, int hd, int rope_pairs, int max_ctx, float eps, int pos0,
                    const int32_t* __restrict__ pos_dev) {
    __shared__ float scratch[4];
    const int h = blockIdx.x, t = blockIdx.y, i = threadIdx.x, half_d = hd >> 1;
    if (pos_dev) pos0 = pos_dev[0];
    const int pos = pos0 + t;
    const bool in_cache = pos >= 0 && pos < max_ctx;
    float* v = qkv + (size_t)t * (n_heads + 2 * n_kv) * hd + (size_t)h * hd;
    const bool live = i < half_d;
    float a = live ? v[i] : 0.0f, b = live ? v[i + half_d] : 0.0f;
    // the head's sum of squares across the workgroup's waves
    float ss = mxd::wave_sum(fmaf(a, a, b * b));
    if ((i & 63) == 0) scratch[i >> 6] = ss;
    __syncthreads();
    ss = scratch[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) ss += scratch[w];
    if (!live) return;
    const float scale = rsqrtf(ss / (float)hd + eps);
    a *= scale;
    b *= scale;
    const int k = pos & 31;
    if (h >= n_heads + n_kv) {  // v: no weight, no rotation
        if (!in_cache) return;
        const int kvh = h - n_heads - n_kv;
        const size_t tile = ((size_t)kvh * max_ctx + (pos & ~31)) * hd;
        vcache[tile + mxd::v_tile_offset(k, i)] = mxd::f2h_bits(a);
        vcache[tile + mxd::v_tile_offset(k, i + half_d)] = mxd::f2h_bits(b);
        return;
    }
    const float* w = h < n_heads ? q_w : k_w;
    a *= w[i];
    b *= w[i + half_d];
    if (i < rope_pairs) {
        const float ang = (float)pos * inv_freq[i];
        float sn, cs;
        sincosf(ang, &sn, &cs);
        const float ra = a * cs - b * sn;
        const float rb = b * cs + a * sn;
        a = ra;
        b = rb;
    }
    if (h < n_heads) {
        v[i] = a;
        v[i + half_d] = b;
    } else if (in_cache) {
        const int kvh = h - n_heads;
        const size_t tile = ((size_t)kvh * max_ctx + (pos & ~31)) * hd;
        kcache[tile + mxd::k_tile_offset(k, i, hd)] = mxd::f2h_bits(a);
        kcache[tile + mxd::k_tile_offset(k, i + half_d, hd)] = mxd::f2h_bits(b);
    }
}

// Prefill's per-layer-embedding gate activation (KG/kernels.metal:451-461):
// dst[t][i] = fp16(gelu_tanh(src[t][i]) * ple[t * ple_stride + i]), i < P.
__global__ void __launch_bounds__(256) ple_gate_act_kernel(const float* __restrict__ src, const float* __restrict__ ple,
                                                           uint16_t* __restrict__ dst, int P, int ple_stride) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= P) return;
    dst[(size_t)t * P + i] = mxd::f2h_bits(mxd::gelu_tanh(src[(size_t)t * P + i]) * ple[(size_t)t * ple_stride + i]);
}

}  // namespace

namespace mxd {

int embed_dev(const uint16_t* E, const int32_t* tokens, int pos, const int32_t* pos_dev, int rows, float* x, int D,
              float scale, int vocab, hipStream_t s, int32_t* step_counter) {
    hipLaunchKernelGGL(embed_kernel, dim3((D + 255) / 256, rows), dim3(256), 0, s, E, tokens, pos, pos_dev, x, D, scale,
                       vocab, step_counter);
    return check_launch("embed");
}

int rope_kv_dev(float* qkv, uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads, int n_kv, int hd,
                int max_ctx, int pos0, int rows, const int32_t* pos_dev, hipStream_t s) {
    const int pairs = (n_heads + n_kv) * (hd / 2);
    hipLaunchKernelGGL(rope_kv_kernel, dim3((pairs + 255) / 256, rows), dim3(256), 0, s, qkv, kcache, vcache, inv_freq,
                       n_heads, n_kv, hd, max_ctx, pos0, pos_dev);
    return check_launch("rope_kv");
}

}  // namespace mxd

extern "C" int mxd_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int rows, int D, float eps,
                           int plus_one, mxd_stream_t stream) {
    MXD_REQUIRE(x && w && y, MXD_ERR_INVALID_ARG, "mxd_rmsnorm: null pointer");
    MXD_REQUIRE(rows > 0 && D > 0, MXD_ERR_INVALID_ARG, "mxd_rmsnorm: rows=%d D=%d must be positive", rows, D);
    hipStream_t s = mxd::as_stream(stream);
    const dim3 grid(rows), block(NORM_THREADS);
    if (y_dtype == MXD_F32) {
        if (plus_one)
            hipLaunchKernelGGL((rmsnorm_kernel<float, true>), grid, block, 0, s, x, w, (float*)y, D, eps);
        else
            hipLaunchKernelGGL((rmsnorm_kernel<float, false>), grid, block, 0, s, x, w, (float*)y, D, eps);
    } else if (y_dtype == MXD_F16) {
        if (plus_one)
            hipLaunchKernelGGL((rmsnorm_kernel<_Float16, true>), grid, block, 0, s, x, w, (_Float16*)y, D, eps);
        else
            hipLaunchKernelGGL((rmsnorm_kernel<_Float16, false>), grid, block, 0, s, x, w, (_Float16*)y, D, eps);
    } else {
        return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_rmsnorm: y_dtype %d", y_dtype);
    }
    return mxd::check_launch("mxd_rmsnorm");
}

extern "C" int mxd_embed(const uint16_t* E, const int32_t* tokens, int pos, int rows, float* x, int D, float scale,
                         int vocab, mxd_stream_t stream) {
    MXD_REQUIRE(E && tokens && x, MXD_ERR_INVALID_ARG, "mxd_embed: null pointer");
    MXD_REQUIRE(pos >= 0 && rows > 0 && D > 0 && vocab > 0, MXD_ERR_INVALID_ARG,
                "mxd_embed: pos=%d rows=%d D=%d vocab=%d", pos, rows, D, vocab);
    return mxd::embed_dev(E, tokens, pos, nullptr, rows, x, D, scale, vocab, mxd::as_stream(stream));
}

extern "C" int mxd_f32_to_f16(const float* src, uint16_t* dst, size_t n, mxd_stream_t stream) {
    if (n == 0) return MXD_OK;
    MXD_REQUIRE(src && dst, MXD_ERR_INVALID_ARG, "mxd_f32_to_f16: null pointer");
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, mxd::as_stream(stream), src, dst, n);
    return mxd::check_launch("mxd_f32_to_f16");
}

extern "C" int mxd_rope_kv(float* qkv, uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads,
                           int n_kv_heads, int head_dim, int max_ctx, int pos0, int rows, mxd_stream_t stream) {
    MXD_REQUIRE(qkv && kcache && vcache && inv_freq, MXD_ERR_INVALID_ARG, "mxd_rope_kv: null pointer");
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && rows > 0 && pos0 >= 0, MXD_ERR_INVALID_ARG,
                "mxd_rope_kv: n_heads=%d n_kv_heads=%d rows=%d pos0=%d", n_heads, n_kv_heads, rows, pos0);
    MXD_REQUIRE(head_dim > 0 && head_dim % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_rope_kv: head_dim=%d must be a multiple of 32 (cache tile layout)", head_dim);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_rope_kv: max_ctx=%d must be a positive multiple of 32", max_ctx);
    MXD_REQUIRE(pos0 + rows <= max_ctx, MXD_ERR_INVALID_ARG, "mxd_rope_kv: positions %d..%d exceed max_ctx %d", pos0,
                pos0 + rows - 1, max_ctx);
    const int pairs = (n_heads + n_kv_heads) * (head_dim / 2);
    (void)pairs;
    return mxd::rope_kv_dev(qkv, kcache, vcache, inv_freq, n_heads, n_kv_heads, head_dim, max_ctx, pos0, rows, nullptr,
                            mxd::as_stream(stream));
}

extern "C" int mxd_rope_kv_paged(float* qkv, uint16_t* kpool, uint16_t* vpool, int n_pages, const float* inv_freq,
                                 int n_heads, int n_kv_heads, int head_dim, const int32_t* page_table, int max_pages,
                                 const int32_t* seq_lens, int n_seqs, mxd_stream_t stream) {
    MXD_REQUIRE(qkv && kpool && vpool && inv_freq && page_table && seq_lens, MXD_ERR_INVALID_ARG,
                "mxd_rope_kv_paged: null pointer");
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_seqs > 0 && n_seqs <= 65535 && n_pages > 0 && max_pages > 0,
                MXD_ERR_INVALID_ARG, "mxd_rope_kv_paged: n_heads=%d n_kv_heads=%d n_seqs=%d n_pages=%d max_pages=%d",
                n_heads, n_kv_heads, n_seqs, n_pages, max_pages);
    MXD_REQUIRE(head_dim > 0 && head_dim % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_rope_kv_paged: head_dim=%d must be a multiple of 32 (page slab layout)", head_dim);
    const int pairs = (n_heads + n_kv_heads) * (head_dim / 2);
    hipLaunchKernelGGL(rope_kv_paged_kernel, dim3((pairs + 255) / 256, n_seqs), dim3(256), 0, mxd::as_stream(stream),
                       qkv, kpool, vpool, inv_freq, n_heads, n_kv_heads, head_dim, page_table, max_pages, seq_lens,
                       n_pages);
    return mxd::check_launch("mxd_rope_kv_paged");
}

extern "C" int mxd_rope_kv_paged_sum(const float* part, int n_splits, float* qkv, uint16_t* kpool, uint16_t* vpool,
                                     int n_pages, const float* inv_freq, int n_heads, int n_kv_heads, int head_dim,
                                     const int32_t* page_table, int max_pages, const int32_t* seq_lens, int n_seqs,
                                     mxd_stream_t stream) {
    MXD_REQUIRE(part && qkv && kpool && vpool && inv_freq && page_table && seq_lens, MXD_ERR_INVALID_ARG,
                "mxd_rope_kv_paged_sum: null pointer");
    MXD_REQUIRE(n_splits >= 1, MXD_ERR_INVALID_ARG, "mxd_rope_kv_paged_sum: n_splits=%d", n_splits);
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_seqs > 0 && n_seqs <= 65535 && n_pages > 0 && max_pages > 0,
                MXD_ERR_INVALID_ARG, "mxd_rope_kv_paged_sum: n_heads=%d n_kv_heads=%d n_seqs=%d n_pages=%d max_pages=%d",
                n_heads, n_kv_heads, n_seqs, n_pages, max_pages);
    MXD_REQUIRE(head_dim > 0 && head_dim % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_rope_kv_paged_sum: head_dim=%d must be a multiple of 32 (page slab layout)", head_dim);
    const int pairs = (n_heads + n_kv_heads) * (head_dim / 2);
    const size_t stride = (size_t)n_seqs * (n_heads + 2 * n_kv_heads) * head_dim;
    return with_splits(n_splits, [&](auto ns) {
        hipLaunchKernelGGL(rope_kv_paged_sum_kernel<decltype(ns)::value>, dim3((pairs + 255) / 256, n_seqs), dim3(256),
                           0, mxd::as_stream(stream), part, n_splits, stride, qkv, kpool, vpool, inv_freq, n_heads,
                           n_kv_heads, head_dim, page_table, max_pages, seq_lens, n_pages);
        return mxd::check_launch("mxd_rope_kv_paged_sum");
    });
}

extern "C" int mxd_rmsnorm_residual_sum(float* x, const float* part, int n_splits, const float* w, void* y,
                                        int y_dtype, int rows, int D, float eps, int plus_one, mxd_stream_t stream) {
    MXD_REQUIRE(x && part && w && y, MXD_ERR_INVALID_ARG, "mxd_rmsnorm_residual_sum: null pointer");
    MXD_REQUIRE(n_splits >= 1, MXD_ERR_INVALID_ARG, "mxd_rmsnorm_residual_sum: n_splits=%d", n_splits);
    MXD_REQUIRE(rows > 0 && D > 0, MXD_ERR_INVALID_ARG, "mxd_rmsnorm_residual_sum: rows=%d D=%d must be positive", rows,
                D);
    MXD_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(w)) &
                 15) == 0,
                MXD_ERR_UNSUPPORTED, "mxd_rmsnorm_residual_sum: x, part and w must be 16-byte aligned");
    MXD_REQUIRE(y_dtype == MXD_F32 || y_dtype == MXD_F16, MXD_ERR_INVALID_ARG, "mxd_rmsnorm_residual_sum: y_dtype %d",
                y_dtype);
    hipStream_t s = mxd::as_stream(stream);
    const dim3 grid(rows), block(NORM_THREADS);
    const size_t stride = (size_t)rows * D;
    // groups per thread of the cached loop: 4 up to D = 4096, 8 up to 8192
    // (rmsnorm_kernel's range), else the plain two-pass loop
    const int nc = D % 4 != 0 ? 0 : D <= 4 * 4 * NORM_THREADS ? 4 : D <= NORM_CACHE * 4 * NORM_THREADS ? 8 : 0;
    auto go = [&](auto ns, auto ncc) {
        constexpr int NS = decltype(ns)::value, NC = decltype(ncc)::value;
        if (y_dtype == MXD_F32) {
            if (plus_one)
                hipLaunchKernelGGL((rmsnorm_residual_sum_kernel<float, true, NS, NC>), grid, block, 0, s, x, part,
                                   n_splits, stride, w, (float*)y, D, eps);
            else
                hipLaunchKernelGGL((rmsnorm_residual_sum_kernel<float, false, NS, NC>), grid, block, 0, s, x, part,
                                   n_splits, stride, w, (float*)y, D, eps);
        } else {
            if (plus_one)
                hipLaunchKernelGGL((rmsnorm_residual_sum_kernel<_Float16, true, NS, NC>), grid, block, 0, s, x, part,
                                   n_splits, stride, w, (_Float16*)y, D, eps);
            else
                hipLaunchKernelGGL((rmsnorm_residual_sum_kernel<_Float16, false, NS, NC>), grid, block, 0, s, x, part,
                                   n_splits, stride, w, (_Float16*)y, D, eps);
        }
        return mxd::check_launch("mxd_rmsnorm_residual_sum");
    };
    return with_splits(n_splits, [&](auto ns) {
        if (nc == 4) return go(ns, std::integral_constant<int, 4>{});
        if (nc == 8) return go(ns, std::integral_constant<int, 8>{});
        return go(ns, std::integral_constant<int, 0>{});
    });
}

// ---- Gemma-4 entry points -------------------------------------------------------

extern "C" int mxd_rmsnorm_add(const float* src, const float* w, float* x, int rows, int D, float eps, float post,
                               mxd_stream_t stream) {
    MXD_REQUIRE(src && w && x, MXD_ERR_INVALID_ARG, "mxd_rmsnorm_add: null pointer");
    MXD_REQUIRE(rows > 0 && D > 0, MXD_ERR_INVALID_ARG, "mxd_rmsnorm_add: rows=%d D=%d must be positive", rows, D);
    hipLaunchKernelGGL(rmsnorm_add_kernel, dim3(rows), dim3(NORM_THREADS), 0, mxd::as_stream(stream), src, w, x, D,
                       eps, post);
    return mxd::check_launch("mxd_rmsnorm_add");
}

extern "C" int mxd_ple_combine(const float* proj, float* ple, const float* w, int rows, int n_layers, int P,
                               float proj_scale, float eps, mxd_stream_t stream) {
    MXD_REQUIRE(proj && ple && w, MXD_ERR_INVALID_ARG, "mxd_ple_combine: null pointer");
    MXD_REQUIRE(rows > 0 && n_layers > 0 && P > 0, MXD_ERR_INVALID_ARG, "mxd_ple_combine: rows=%d n_layers=%d P=%d",
                rows, n_layers, P);
    hipLaunchKernelGGL(ple_combine_kernel, dim3(n_layers, rows), dim3(NORM_THREADS), 0, mxd::as_stream(stream), proj,
                       ple, w, P, n_layers * P, proj_scale, eps);
    return mxd::check_launch("mxd_ple_combine");
}

extern "C" int mxd_qk_norm_rope_kv(float* qkv, uint16_t* kcache, uint16_t* vcache, const float* q_w, const float* k_w,
                                   const float* inv_freq, int n_heads, int n_kv_heads, int head_dim, int rope_pairs,
                                   int max_ctx, float eps, int pos0, int rows, const int32_t* pos_dev,
                                   mxd_stream_t stream) {
    MXD_REQUIRE(qkv && q_w && inv_freq, MXD_ERR_INVALID_ARG, "mxd_qk_norm_rope_kv: null pointer");
    MXD_REQUIRE(n_heads > 0 && n_kv_heads >= 0 && rows > 0, MXD_ERR_INVALID_ARG,
                "mxd_qk_norm_rope_kv: n_heads=%d n_kv_heads=%d rows=%d", n_heads, n_kv_heads, rows);
    MXD_REQUIRE(n_kv_heads == 0 || (kcache && vcache && k_w), MXD_ERR_INVALID_ARG,
                "mxd_qk_norm_rope_kv: kv heads need caches and k_w");
    MXD_REQUIRE(head_dim >= 32 && head_dim <= 512 && head_dim % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_qk_norm_rope_kv: head_dim %d (a multiple of 32 up to 512)", head_dim);
    MXD_REQUIRE(rope_pairs >= 0 && rope_pairs <= head_dim / 2, MXD_ERR_INVALID_ARG,
                "mxd_qk_norm_rope_kv: rope_pairs %d outside [0, %d]", rope_pairs, head_dim / 2);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED, "mxd_qk_norm_rope_kv: max_ctx=%d", max_ctx);
    MXD_REQUIRE(pos_dev || (pos0 >= 0 && (n_kv_heads == 0 || pos0 + rows <= max_ctx)), MXD_ERR_INVALID_ARG,
                "mxd_qk_norm_rope_kv: positions [%d, %d) outside [0, %d)", pos0, pos0 + rows, max_ctx);
    const int threads = (head_dim / 2 + 63) / 64 * 64;
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(n_heads + 2 * n_kv_heads, rows), dim3(threads), 0,
                       mxd::as_stream(stream), qkv, kcache, vcache, q_w, k_w, inv_freq, n_heads, n_kv_heads, head_dim,
                       rope_pairs, max_ctx, eps, pos0, pos_dev);
    return mxd::check_launch("mxd_qk_norm_rope_kv");
}

extern "C" int mxd_ple_gate_act(const float* src, const float* ple, uint16_t* dst, int rows, int P, int ple_stride,
                                mxd_stream_t stream) {
    MXD_REQUIRE(src && ple && dst, MXD_ERR_INVALID_ARG, "mxd_ple_gate_act: null pointer");
    MXD_REQUIRE(rows > 0 && P > 0 && ple_stride >= P, MXD_ERR_INVALID_ARG,
                "mxd_ple_gate_act: rows=%d P=%d ple_stride=%d", rows, P, ple_stride);
    hipLaunchKernelGGL(ple_gate_act_kernel, dim3((P + 255) / 256, rows), dim3(256), 0, mxd::as_stream(stream), src, ple,
                       dst, P, ple_stride);
    return mxd::check_launch("mxd_ple_gate_act");
}
