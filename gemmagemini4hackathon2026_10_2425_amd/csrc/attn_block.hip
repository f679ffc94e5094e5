// The attention half of a decode layer in one launch:
//
//   [q | k | v] = Wqkv . rmsnorm(x)          (phase 1: matvec, fused norm)
//   RoPE on q and k at pos; k, v -> caches   (phase 1 epilogue)
//   att = softmax(q K^T * scale) V           (phase 2: split attention + merge)
//   x  += Wo . att                           (phase 3: matvec, residual add)
//
// the reference's rmsnorm / matvec(wqkv) / rope_kv / attention / matvec_add(wo)
// chain (KL/main.swift:333-337), which the unfused engine runs as three
// launches (qkv + RoPE, attention split, o projection with the merge). Each
// launch on MI355X costs a fixed ~3.5 us (dispatch, the first HBM round trip,
// the drain) on top of its bytes; this chain moves only ~19 MB per Gemma-2B
// layer, so the fixed costs dominated it.
//
// One grid, three phases by workgroup id (producers first):
//   [0, n1)            phase 1: NR1 virtual rows of the q|k|v projection each
//   [n1, n1 + n2)      phase 2: split s of kv head h (id n1 + s * n_kv + h,
//                      s < s_max), then 256-value slices of the log-sum-exp
//                      merge of the splits
//   [n1 + n2, ...)     phase 3: NR rows of the o projection each
// Values pass between workgroups as tagged words (common.hpp): q, k and v from
// phase 1, the split partials and the merged attention output from phase 2.
// A workgroup only ever waits for workgroups with smaller ids, and the
// dispatcher starts workgroups in id order, so every wait ends even when the
// grid does not fit the GPU at once; waits are also bounded (a stuck wait
// sets the error word). Phase 2 issues its first K/V block loads and phase 3
// its weight loads before they wait.
//
// The tag of a launch is step * 64 + layer, step read from a device counter
// the caller advances once per decode step (the engine's embedding kernel
// does), so no two launches that share the workspace use the same tag.
//
// Measured on MI355X (Gemma-2B layer, 160 + 11 + 128 workgroups at one per CU):
// phase 1 is done by ~6.5 us, but each handoff between XCDs then costs 1-12
// us before the consumer holds its words (agent-scope stores and loads, or
// read-modify-write atomics, alike; sparser polling changes nothing), and the
// launch takes ~31 us against 18.8 us for the three launches it replaces, so
// the engine runs it only under the ENG_FUSED tunable.
#include "attn_core.hpp"
#include "gemv_core.hpp"

namespace {

constexpr int AB_W = 4;  // waves per workgroup
constexpr int AB_MAX_LAYERS = 64;

// Rows per workgroup of phases 1 and 3. The attention phase sets the kernel's
// registers: at head_dim 256 one wave per SIMD fits (one workgroup per CU), so
// the matvec phases take 16 rows per workgroup there to stay within about one
// round of workgroups; smaller heads take 8.
template <int HD> struct ABRows { static constexpr int NR = HD == 256 ? 16 : 8; };

struct BlockArgs {
    const uint16_t* wqkv;
    const uint16_t* wo;
    float* x;  // residual, read by phase 1, updated by phase 3
    const float* norm_w;
    float eps;
    int plus_one;
    uint16_t* kcache;
    uint16_t* vcache;
    const float* inv_freq;
    int n_heads, n_kv, hd, dim, max_ctx;
    int pos;
    const int32_t* pos_dev;
    float qscale;  // scale * log2(e)
    const int32_t* step_dev;
    int layer;
    int n1, n2, n3, s_max;
    // workspace (tagged words)
    uint64_t* tq;    // [n_heads * hd]
    uint64_t* tk;    // [n_kv * hd]
    uint64_t* tv;    // [n_kv * hd]
    uint64_t* tpo;   // [s_max][n_heads][hd]
    uint64_t* tpml;  // [s_max][n_heads][2]
    uint64_t* tatt;  // [n_heads * hd]
    int* err;
};

__device__ __forceinline__ int block_pos(const BlockArgs& b) {
    const int p = b.pos_dev ? b.pos_dev[0] : b.pos;
    return max(0, min(p, b.max_ctx - 1));
}

// Splits active at n keys: one 32-key block per wave, at most s_max.
__device__ __forceinline__ int block_splits(const BlockArgs& b, int n) {
    const int nblocks = (n + BLK - 1) / BLK;
    return max(1, min(b.s_max, (nblocks + AB_W - 1) / AB_W));
}

// ---- phase 1: q|k|v rows with the fused norm, RoPE and the cache append ----
template <int NR>
__device__ __forceinline__ void phase_qkv(const BlockArgs& b, int wg, uint32_t tag, int pos) {
    constexpr int EPL = 8, CH = 64 * EPL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = b.dim, nch = (K + CH - 1) / CH;
    const int M = (b.n_heads + 2 * b.n_kv) * b.hd;
    const int r0 = wg * NR;
    GemvArgs ga{};
    ga.n_heads = b.n_heads;
    ga.n_kv = b.n_kv;
    ga.hd = b.hd;
    const unsigned char* wrow[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int row = rope_row(min(r0 + r, M - 1), ga);
        wrow[r] = reinterpret_cast<const unsigned char*>(b.wqkv) + (size_t)row * K * 2;
    }
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
    for (int c = wave; c < nch; c += AB_W) {
        const int col = c * CH + lane * EPL;
        if (col >= K) continue;
        u4_t wv[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) wv[r] = ld_stream<MXD_W_F16>(wrow[r] + (size_t)col * 2);
        XFrag<float, EPL> xf;
        xf.load_norm(b.x, b.norm_w, col, 1.0f, b.plus_one);
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = dot16(wv[r], xf, acc[r]);
    }
    const float nscale = block_rms_scale<AB_W>(b.x, K, b.eps);
    __shared__ float red[AB_W][NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = mxd::wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) red[wave][r] = acc[r];
    }
    __syncthreads();
    // Rows r0 .. r0 + NR - 1 in rotation pairs: thread p < NR / 2 of wave 0
    // finishes pair p (angle pos * inv_freq[i] in fp32, accurate sin/cos), as
    // the unfused projection's epilogue does (KL/kernels.metal:199-222).
    if (wave != 0 || lane >= NR / 2) return;
    const int r = 2 * lane, v = r0 + r;
    if (v >= M) return;
    float s0 = red[0][r], s1 = red[0][r + 1];
#pragma unroll
    for (int w = 1; w < AB_W; ++w) {
        s0 += red[w][r];
        s1 += red[w][r + 1];
    }
    s0 *= nscale;
    s1 *= nscale;
    const int hd = b.hd, half = hd >> 1, qk_rows = (b.n_heads + b.n_kv) * hd, kpos = pos & 31;
    if (v < qk_rows) {
        const int p = v >> 1, head = p / half, i = p - head * half;
        const float ang = (float)pos * b.inv_freq[i];
        float sn, cs;
        sincosf(ang, &sn, &cs);
        const float ra = s0 * cs - s1 * sn;
        const float rb = s1 * cs + s0 * sn;
        if (head < b.n_heads) {
            mxd::tag_put(b.tq + head * hd + i, tag, ra);
            mxd::tag_put(b.tq + head * hd + i + half, tag, rb);
        } else {
            const int kvh = head - b.n_heads;
            const size_t tile = ((size_t)kvh * b.max_ctx + (pos & ~31)) * hd;
            b.kcache[tile + mxd::k_tile_offset(kpos, i, hd)] = mxd::f2h_bits(ra);
            b.kcache[tile + mxd::k_tile_offset(kpos, i + half, hd)] = mxd::f2h_bits(rb);
            mxd::tag_put(b.tk + kvh * hd + i, tag, ra);
            mxd::tag_put(b.tk + kvh * hd + i + half, tag, rb);
        }
    } else {
        const float vals[2] = {s0, s1};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            if (v + e >= M) break;
            const int vr = v + e - qk_rows, kvh = vr / hd, d = vr - kvh * hd;
            const size_t tile = ((size_t)kvh * b.max_ctx + (pos & ~31)) * hd;
            b.vcache[tile + mxd::v_tile_offset(kpos, d)] = mxd::f2h_bits(vals[e]);
            mxd::tag_put(b.tv + vr, tag, vals[e]);
        }
    }
}

// Merge slice m: value idx = m * 256 + thread of the n_heads * HD outputs, the
// log-sum-exp combination of the S partials of its head (nothing to do for a
// single split, which wrote the output itself); each wait takes eight
// splits' (max, sum, O) words at once. These workgroups come after every
// split's, so they only wait for smaller ids.
template <int HD>
__device__ __forceinline__ void merge_slice(const BlockArgs& b, int m, int S, uint32_t tag) {
    if (S == 1) return;
    const int total = b.n_heads * HD;
    const int idx = m * AB_W * 64 + (int)threadIdx.x;
    if (idx >= total) return;
    const int h = idx / HD;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 8) {
        const uint64_t* p[24];
        float v[24];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bool live = s0 + i < S;
            const size_t row = (size_t)(s0 + i) * b.n_heads + h;
            p[i] = live ? b.tpml + row * 2 : nullptr;
            p[8 + i] = live ? b.tpml + row * 2 + 1 : nullptr;
            p[16 + i] = live ? b.tpo + (size_t)(s0 + i) * total + idx : nullptr;
        }
        mxd::tag_wait<24>(p, tag, v, b.err);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (s0 + i >= S) break;
            const float Mn = fmaxf(M, v[i]);
            const float fa = __builtin_amdgcn_exp2f(M - Mn), fb = __builtin_amdgcn_exp2f(v[i] - Mn);
            L = L * fa + v[8 + i] * fb;
            O = O * fa + v[16 + i] * fb;
            M = Mn;
        }
    }
    mxd::tag_put(b.tatt + idx, tag, O / L);
}

// ---- phase 2: one split of one kv head (or a merge slice) --------------
template <int HD>
__device__ __forceinline__ void phase_attention(const BlockArgs& b, int j, uint32_t tag, int pos) {
    const int n = pos + 1, nblocks = (n + BLK - 1) / BLK;
    const int S = block_splits(b, n);
    const int n_split_wgs = b.s_max * b.n_kv;
    const int G = b.n_heads / b.n_kv;
    if (j >= n_split_wgs) {
        merge_slice<HD>(b, j - n_split_wgs, S, tag);
        return;
    }
    const int s = j / b.n_kv, kvh = j - s * b.n_kv;
    AttnArgs a{};
    a.k = b.kcache;
    a.v = b.vcache;
    a.n_heads = b.n_heads;
    a.n_kv = b.n_kv;
    a.G = G;
    a.max_ctx = b.max_ctx;
    a.qscale = b.qscale;
    a.tq = b.tq;
    a.tk = b.tk;
    a.tv = b.tv;
    a.tag = tag;
    a.patch_pos = pos;
    a.err = b.err;
    if (s < S) {
        const ContigKV<HD> src{b.kcache + (size_t)kvh * b.max_ctx * HD, b.vcache + (size_t)kvh * b.max_ctx * HD};
        const size_t g0 = (size_t)kvh * G;
        CoreOut out{nullptr, nullptr, nullptr, S == 1};
        if (S == 1) {
            out.trow = b.tatt + g0 * HD;
        } else {
            const size_t prow = (size_t)s * b.n_heads + g0;
            out.trow = b.tpo + prow * HD;
            out.tml = b.tpml + prow * 2;
        }
        attn_core<HD, AB_W, false, ContigKV<HD>, true>(a, src, n, s, S, nblocks, nullptr, out, kvh);
    }
}

// ---- phase 3: o-projection rows with the residual add ----------------------
template <int NR, int MAXC>
__device__ __forceinline__ void phase_oproj(const BlockArgs& b, int wg, uint32_t tag) {
    constexpr int EPL = 8, CH = 64 * EPL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = b.n_heads * b.hd, nch = (K + CH - 1) / CH, D = b.dim;
    const int r0 = wg * NR;
    // This wave's chunks wave, wave + 4, ... (MAXC of them): all weight loads
    // go out before the wait for the attention output.
    u4_t wv[MAXC][NR];
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
        const int c = wave + u * AB_W, col = c * CH + lane * EPL;
        if (c >= nch || col >= K) continue;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int row = min(r0 + r, D - 1);
            wv[u][r] = ld_stream<MXD_W_F16>(reinterpret_cast<const unsigned char*>(b.wo) + ((size_t)row * K + col) * 2);
        }
    }
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
        const int c = wave + u * AB_W, col = c * CH + lane * EPL;
        if (c >= nch || col >= K) continue;
        const uint64_t* p[EPL];
        XFrag<float, EPL> xf;
#pragma unroll
        for (int e = 0; e < EPL; ++e) p[e] = b.tatt + col + e;
        mxd::tag_wait<EPL>(p, tag, xf.v, b.err);
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = dot16(wv[u][r], xf, acc[r]);
    }
    __shared__ float red3[AB_W][NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = mxd::wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) red3[wave][r] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < NR && r0 + (int)threadIdx.x < D) {
        const int r = threadIdx.x;
        float s = red3[0][r];
#pragma unroll
        for (int w = 1; w < AB_W; ++w) s += red3[w][r];
        b.x[r0 + r] += s;
    }
}

template <int HD, int CPW3>
__global__ void __launch_bounds__(AB_W * 64) attn_block_kernel(BlockArgs b) {
    constexpr int NR = ABRows<HD>::NR;
    const uint32_t tag = (uint32_t)b.step_dev[0] * (uint32_t)AB_MAX_LAYERS + (uint32_t)b.layer;
    const int pos = block_pos(b);
    const int id = blockIdx.x;
    if (id < b.n1)
        phase_qkv<NR>(b, id, tag, pos);
    else if (id < b.n1 + b.n2)
        phase_attention<HD>(b, id - b.n1, tag, pos);
    else
        phase_oproj<NR, CPW3>(b, id - b.n1 - b.n2, tag);
}

template <int HD>
void launch_block(const BlockArgs& b, hipStream_t s) {
    const dim3 grid(b.n1 + b.n2 + b.n3), block(AB_W * 64);
    const int nch3 = (b.n_heads * b.hd + 511) / 512;  // o-projection chunks of 512 columns
    const int cpw = (nch3 + AB_W - 1) / AB_W;
    if (cpw <= 1)
        hipLaunchKernelGGL((attn_block_kernel<HD, 1>), grid, block, 0, s, b);
    else if (cpw <= 2)
        hipLaunchKernelGGL((attn_block_kernel<HD, 2>), grid, block, 0, s, b);
    else
        hipLaunchKernelGGL((attn_block_kernel<HD, 4>), grid, block, 0, s, b);
}

// Splits of the largest context (one block per wave), as the device's
// block_splits caps them: enough workgroups to cover ~3 per CU in all.
int block_s_max(int max_ctx, int n_kv) {
    const int nblocks = (max_ctx + BLK - 1) / BLK;
    const int per_cu = max(1, min(16, mxd::tunable("AB_WGCU", 3)));
    const int cap = min(512, (per_cu * 256 + n_kv - 1) / n_kv);
    return max(1, min(cap, (nblocks + AB_W - 1) / AB_W));
}

size_t ws_words(int n_heads, int n_kv, int hd, int s_max) {
    const size_t q = (size_t)n_heads * hd, kv = (size_t)n_kv * hd;
    return q + 2 * kv + (size_t)s_max * q + (size_t)s_max * n_heads * 2 + q;
}

}  // namespace

namespace mxd {

size_t attn_block_workspace_size(int n_heads, int n_kv, int hd, int max_ctx) {
    return ws_words(n_heads, n_kv, hd, block_s_max(max_ctx, n_kv)) * 8 + 256;
}

int attn_block(const uint16_t* wqkv, const uint16_t* wo, float* x, const float* norm_w, float eps, int plus_one,
               uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads, int n_kv, int hd, int dim,
               int max_ctx, int pos, const int32_t* pos_dev, float scale, const int32_t* step_dev, int layer,
               void* workspace, size_t ws_bytes, hipStream_t s) {
    MXD_REQUIRE(wqkv && wo && x && norm_w && kcache && vcache && inv_freq && step_dev && workspace,
                MXD_ERR_INVALID_ARG, "attn_block: null pointer");
    MXD_REQUIRE(n_heads > 0 && n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= 8, MXD_ERR_UNSUPPORTED,
                "attn_block: n_heads=%d n_kv=%d (group of 1..8)", n_heads, n_kv);
    MXD_REQUIRE(hd == 64 || hd == 128 || hd == 256, MXD_ERR_UNSUPPORTED, "attn_block: head_dim %d", hd);
    MXD_REQUIRE(dim > 0 && dim % 8 == 0 && (n_heads * hd) <= 4 * AB_W * 512, MXD_ERR_UNSUPPORTED,
                "attn_block: dim=%d, n_heads * head_dim=%d (at most 8192)", dim, n_heads * hd);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED, "attn_block: max_ctx=%d", max_ctx);
    MXD_REQUIRE(layer >= 0 && layer < AB_MAX_LAYERS, MXD_ERR_UNSUPPORTED, "attn_block: layer %d (at most %d)", layer,
                AB_MAX_LAYERS);
    MXD_REQUIRE(pos_dev || (pos >= 0 && pos < max_ctx), MXD_ERR_INVALID_ARG, "attn_block: pos %d", pos);
    const int s_max = block_s_max(max_ctx, n_kv);
    const size_t words = ws_words(n_heads, n_kv, hd, s_max);
    MXD_REQUIRE(ws_bytes >= words * 8 + 256, MXD_ERR_WORKSPACE, "attn_block: workspace of %zu bytes needed",
                words * 8 + 256);
    BlockArgs b{};
    b.wqkv = wqkv;
    b.wo = wo;
    b.x = x;
    b.norm_w = norm_w;
    b.eps = eps;
    b.plus_one = plus_one;
    b.kcache = kcache;
    b.vcache = vcache;
    b.inv_freq = inv_freq;
    b.n_heads = n_heads;
    b.n_kv = n_kv;
    b.hd = hd;
    b.dim = dim;
    b.max_ctx = max_ctx;
    b.pos = pos;
    b.pos_dev = pos_dev;
    b.qscale = scale * LOG2E;
    b.step_dev = step_dev;
    b.layer = layer;
    b.s_max = s_max;
    const int nr = hd == 256 ? ABRows<256>::NR : ABRows<128>::NR;
    b.n1 = ((n_heads + 2 * n_kv) * hd + nr - 1) / nr;
    // phase 2: the splits of every kv head, then one merge thread per
    // attention output
    b.n2 = s_max * n_kv + (n_heads * hd + AB_W * 64 - 1) / (AB_W * 64);
    b.n3 = (dim + nr - 1) / nr;
    uint64_t* w = static_cast<uint64_t*>(workspace);
    const size_t q = (size_t)n_heads * hd, kv = (size_t)n_kv * hd;
    b.tq = w;
    b.tk = b.tq + q;
    b.tv = b.tk + kv;
    b.tpo = b.tv + kv;
    b.tpml = b.tpo + (size_t)s_max * q;
    b.tatt = b.tpml + (size_t)s_max * n_heads * 2;
    b.err = reinterpret_cast<int*>(b.tatt + q);
    if (hd == 64)
        launch_block<64>(b, s);
    else if (hd == 128)
        launch_block<128>(b, s);
    else
        launch_block<256>(b, s);
    return check_launch("attn_block");
}

// The error word of an attn_block workspace: set when a wait ran out.
int* attn_block_err(void* workspace, int n_heads, int n_kv, int hd, int max_ctx) {
    const size_t words = ws_words(n_heads, n_kv, hd, block_s_max(max_ctx, n_kv));
    return reinterpret_cast<int*>(static_cast<uint64_t*>(workspace) + words);
}

}  // namespace mxd
