// Device core of single-query attention on the matrix cores, shared by the
// attention kernels (attention.hip) and the fused decode attention block
// (attn_block.hip): the argument block, the 32-key K/V block loaders of the
// contiguous and paged caches, and one kv head's online-softmax walk over
// its blocks.
#pragma once

#include "common.hpp"

namespace {

constexpr int ATT_WAVES = 4;  // default waves per workgroup
constexpr int BLK = 32;  // keys per wave step
constexpr int MAX_SPLITS = 512;
constexpr int PAGED_BPS = 16;  // default 32-key blocks per split of a paged sequence (4 per wave)
constexpr float LOG2E = 1.4426950408889634f;
// Balanced paged schedule: at most SK_MAX_SEQS sequences (their block prefix
// lives in LDS), and at least SK_MIN_BLOCKS blocks per workgroup.
constexpr int SK_MAX_SEQS = 2048;
constexpr int SK_MIN_BLOCKS = 8;

struct AttnArgs {
    const float* q;
    const uint16_t* k;  // contiguous tiled cache, or the page pool
    const uint16_t* v;
    float* out;
    // prefill: the output rows in fp16 instead (out's strides), rounded to
    // nearest even as mxd_f32_to_f16 rounds
    uint16_t* out_h = nullptr;
    float* ws_o;   // [seqs][n_splits][n_heads][HD]
    float* ws_ml;  // [seqs][n_splits][n_heads][2]
    const int32_t* pos_dev;
    // paged: page_table [seqs][max_pages] of pool pages, seq_lens [seqs] keys
    const int32_t* page_table = nullptr;
    const int32_t* seq_lens = nullptr;
    int max_pages = 0, n_pages = 0, q_stride = 0, out_stride = 0, bps = PAGED_BPS;
    // paged, balanced schedule: sequences, workgroups launched, and the
    // per-sequence block prefix the attention kernel leaves for the merge
    int n_seqs = 0, sk_wgs = 0;
    int32_t* sk_pre = nullptr;
    int n_heads, n_kv, G, max_ctx, n_keys, n_splits;
    float qscale;  // scale * log2(e): scores live in the log2 domain
    // Every active split leaves a partial, also a single one (the consumer
    // merges them): mxd_attention_split.
    bool partials_only = false;
    // mxd_attention: the splits that take blocks follow from the key count on
    // the device (active_splits), so a grid sized for max_ctx under a device
    // position splits a given context exactly as a launch for that context.
    bool auto_splits = false;
    int single_blocks = 0;  // contexts of up to this many blocks take one split
    int waves = 4;
    // Sliding window (contiguous cache): a query with n visible keys attends to
    // keys [max(0, n - window), n); 0 = all n.
    int window = 0;
    // Tagged mode (the fused decode attention block): the q rows ([n_heads][HD])
    // and the new key / value rows of position patch_pos ([n_kv][HD], fp32
    // before their fp16 rounding) arrive as tagged words of `tag`; the block of
    // patch_pos takes them in place of what its cache lines held (another XCD
    // wrote them in this launch), and the core's results leave as tagged words.
    const uint64_t* tq = nullptr;
    const uint64_t* tk = nullptr;
    const uint64_t* tv = nullptr;
    uint32_t tag = 0;
    int patch_pos = -1;
    int* err = nullptr;
};

// Keys visible to the query: n_keys, or *pos_dev + 1 read on the device (clamped
// to the cache so a bad position can never address past it).
__device__ __forceinline__ int n_keys_of(const AttnArgs& a) {
    const int n = a.pos_dev ? a.pos_dev[0] + 1 : a.n_keys;
    return max(0, min(n, a.max_ctx));
}

// First key a query with n visible keys attends to.
__device__ __forceinline__ int window_lo(const AttnArgs& a, int n) { return a.window > 0 ? max(0, n - a.window) : 0; }

// 32-key blocks holding the keys [window_lo, n).
__device__ __forceinline__ int attended_blocks(const AttnArgs& a, int n) {
    return (n + BLK - 1) / BLK - window_lo(a, n) / BLK;
}

// Splits of a context of nblocks 32-key blocks under auto_splits: one up to
// single_blocks, else one block per wave, capped by the launched grid. The
// host's splits_for computes the grid with the same rule.
__device__ __forceinline__ int active_splits(const AttnArgs& a, int nblocks) {
    if (!a.auto_splits) return a.n_splits;
    if (nblocks <= a.single_blocks) return 1;
    return min(a.n_splits, (nblocks + a.waves - 1) / a.waves);
}

template <int HD>
struct KVBlock {
    h8_t k[2][HD / 32];
    h8_t v[HD / 16];
};

// Loads of one 32-key block starting at key0 (a multiple of 32). The caches
// are stored in MFMA operand order (the tile layouts in include/mxdecode.h),
// so every operand is one 1 KiB contiguous wave load: lane l reads the 16
// bytes at l * 16 of its chunk. K chunk (t, c) holds, for lane (col, g), key
// 8(col>>2) + 4t + (col&3) of the block and dims 32c + 8g .. +7 (row 4g'+i of
// S^T tile t is then key 8g' + 4t + i); V chunk d holds keys 8g .. +7 of dim
// 16d + col.
template <int HD>
__device__ __forceinline__ void load_block(KVBlock<HD>& kv, const uint16_t* kbase, const uint16_t* vbase, int key0,
                                           int lane) {
    const uint16_t* kt = kbase + (size_t)key0 * HD + 8 * lane;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < HD / 32; ++c)
            kv.k[t][c] = __builtin_nontemporal_load(reinterpret_cast<const h8_t*>(kt + (t * (HD / 32) + c) * 512));
    const uint16_t* vt = vbase + (size_t)key0 * HD + 8 * lane;
#pragma unroll
    for (int d = 0; d < HD / 16; ++d) kv.v[d] = __builtin_nontemporal_load(reinterpret_cast<const h8_t*>(vt + d * 512));
}

// A contiguous (tiled) cache of one kv head.
template <int HD>
struct ContigKV {
    const uint16_t* kbase;
    const uint16_t* vbase;
    using Addr = int;  // the block index
    __device__ __forceinline__ Addr addr(int b) const { return b; }
    __device__ __forceinline__ void load(KVBlock<HD>& kv, Addr b, int lane) const {
        load_block<HD>(kv, kbase, vbase, b * BLK, lane);
    }
    // Key (within the block) of score slot j of lane group g; the same slot
    // order is the k order of the P.V operands.
    static __device__ __forceinline__ int key(int g, int j) { return 8 * g + j; }
};

// One sequence's pages of one kv head in the page pool (slab layouts in
// common.hpp). Block b is pages 2b (keys 0..15 of the block) and 2b + 1 (keys
// 16..31): a slab holds that half of the contiguous tile, so the key of each
// score slot is the same as in ContigKV and only the addresses differ. Lanes
// with col < 8 read K from the first page, lane groups g < 2 read V from it.
template <int HD>
struct PagedKV {
    const uint16_t* kpool;
    const uint16_t* vpool;
    const int32_t* table;  // this sequence's page-table row
    int npages;            // pages holding its keys
    int n_pages;           // pages in the pool
    size_t page_stride;    // n_kv * PAGE_KEYS * HD halfs
    int kvh;
    __device__ __forceinline__ size_t slab(int logical) const {
        int p = table[logical];
        p = p < 0 ? 0 : (p >= n_pages ? n_pages - 1 : p);  // a bad entry still addresses inside the pool
        return (size_t)p * page_stride + (size_t)kvh * mxd::PAGE_KEYS * HD;
    }
    // The block's two slabs, looked up in the page table. The core asks for
    // the next block's address one iteration early, so the table read is off
    // the path of the K/V loads. A ragged last block has one page: its second
    // half re-reads the first page, and every key of it is masked.
    struct Addr {
        size_t s0, s1;
    };
    __device__ __forceinline__ Addr addr(int b) const { return Addr{slab(2 * b), slab(min(2 * b + 1, npages - 1))}; }
    __device__ __forceinline__ void load(KVBlock<HD>& kv, const Addr& ad, int lane) const {
        const size_t s0 = ad.s0, s1 = ad.s1;
        const int col = lane & 15, g = lane >> 4;
        const uint16_t* kp = kpool + ((col >> 3) ? s1 : s0) + (size_t)(g * 8 + (col & 7)) * 8;
        const uint16_t* vp = vpool + ((g >> 1) ? s1 : s0) + (size_t)((g & 1) * 16 + col) * 8;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int c = 0; c < HD / 32; ++c)
                kv.k[t][c] = __builtin_nontemporal_load(reinterpret_cast<const h8_t*>(kp + (c * 2 + t) * 256));
#pragma unroll
        for (int d = 0; d < HD / 16; ++d)
            kv.v[d] = __builtin_nontemporal_load(reinterpret_cast<const h8_t*>(vp + d * 256));
    }
    static __device__ __forceinline__ int key(int g, int j) { return 8 * g + j; }
};

// Where one run of the core leaves its result: the normalised output rows of
// the kv head's G query heads ([G][HD]), or an unnormalised partial, O rows
// [G][HD] plus (max, sum) pairs [G][2], for a later log-sum-exp merge.
struct CoreOut {
    float* orow;
    float* po;
    float* pml;
    bool direct;
    // tagged mode: the same values as tagged words (rows, then (max, sum) pairs)
    uint64_t* trow = nullptr;
    uint64_t* tml = nullptr;
    // a direct output in fp16 at these rows instead of orow
    uint16_t* orow_h = nullptr;
};

// Tagged mode: put the new key and value of position a.patch_pos (fp16 of the
// fp32 rows staged in LDS) into the registers of the block that holds it, at
// the slots the operand layouts give them (K chunk (t, c): lane (col, g)
// holds key 8 (col >> 2) + 4 t + (col & 3), dims 32 c + 8 g .. + 7; V chunk
// d: lane (col, g) holds keys 8 g .. 8 g + 7 of dim 16 d + col). Element
// indices stay compile-time constants (a runtime index into a vector register
// would go through scratch memory): every slot is rewritten with a select.
template <int HD>
__device__ __forceinline__ void patch_block(const AttnArgs& a, KVBlock<HD>& kv, const float* knew, const float* vnew,
                                            int lane) {
    constexpr int NC = HD / 32, ND = HD / 16;
    const int col = lane & 15, g = lane >> 4, kp = a.patch_pos & 31;
    const int tk = (kp >> 2) & 1, jv = kp & 7;
    const bool kown = ((col >> 2) == (kp >> 3)) && ((col & 3) == (kp & 3));
    const bool vown = g == (kp >> 3);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                kv.k[t][c][e] = (kown && t == tk) ? (_Float16)knew[32 * c + 8 * g + e] : kv.k[t][c][e];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int j = 0; j < 8; ++j) kv.v[d][j] = (vown && j == jv) ? (_Float16)vnew[16 * d + col] : kv.v[d][j];
}

// Tagged mode: the workgroup stages the q rows of its G heads and the new key
// and value rows of its kv head from their tagged words into LDS, every
// thread's words loaded at once (one round trip once they are there).
template <int HD, int NT>
__device__ __forceinline__ void stage_tagged(const AttnArgs& a, int kvh, float* sq, float* sk, float* sv) {
    const int G = a.G;
    constexpr int PER = (8 * HD + 2 * HD + NT - 1) / NT;  // words per thread, G <= 8
    const int nq = G * HD, total = nq + 2 * HD;
    const uint64_t* p[PER];
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = (int)threadIdx.x + i * NT;
        p[i] = idx >= total ? nullptr
               : idx < nq   ? a.tq + (size_t)kvh * G * HD + idx
               : idx < nq + HD ? a.tk + (size_t)kvh * HD + (idx - nq)
                               : a.tv + (size_t)kvh * HD + (idx - nq - HD);
    }
    mxd::tag_wait<PER>(p, a.tag, v, a.err);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = (int)threadIdx.x + i * NT;
        if (idx >= total) break;
        if (idx < nq)
            sq[idx] = v[i];
        else if (idx < nq + HD)
            sk[idx - nq] = v[i];
        else
            sv[idx - nq - HD] = v[i];
    }
    __syncthreads();
}

// One kv head of one sequence with n keys, over the 32-key blocks first,
// first + S, first + 2S, ... below bend, dealt round-robin to the W waves
// (wave w takes first + S*w, then steps by S*W). qg points at the q rows of
// the kv head's G query heads. The range must hold at least one block. Keys
// below lo (a sliding window's start) are masked like keys past n.
template <int HD, int W, bool PREFETCH, typename KV, bool TAGGED = false>
__device__ __forceinline__ void attn_core(const AttnArgs& a, const KV& src, int n, int first, int S, int bend,
                                          const float* qg, const CoreOut& out, int kvh = 0, int lo = 0) {
    constexpr int NC = HD / 32;  // MFMA k-chunks over head_dim for Q.K
    constexpr int ND = HD / 16;  // 16-wide dim tiles for P.V
    constexpr int NT = W * 64;
    // per-wave O: [wave][row][dim], rows 0-7 the hi part of heads 0-7, rows
    // 8-15 the lo part (summed in the merge); rows padded by 4 floats so both
    // the tile writes and the merge's reads hit distinct banks
    __shared__ float sm_o[W][16][HD + 4];
    __shared__ float sm_m[W][8];
    __shared__ float sm_l[W][8];
    __shared__ float sm_c[W][8];  // merge weight of wave w for head h
    // tagged mode: q rows of the G heads, the new key and value rows
    __shared__ float sm_tq[TAGGED ? 8 * HD : 1];
    __shared__ float sm_tk[TAGGED ? HD : 1];
    __shared__ float sm_tv[TAGGED ? HD : 1];

    const int G = a.G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;

    // With S splits of a kv head, split s owning blocks s, s+S, ..., the
    // splits stream one contiguous run of the cache at any moment. The first
    // block's loads go out before the q operand is built so the two latencies
    // overlap.
    const int nblocks = bend;
    const int step = S * W;
    int b = first + S * wave;
    KVBlock<HD> cur, nxt;
    if (b < nblocks) src.load(cur, src.addr(b), lane);

    // Q^T operand: column h holds fp16(q) of head kvh*G + h and column h + 8
    // the remainder fp16(q - hi) (h < G <= 8); the rest are zero. k-slot (g, j)
    // of chunk c is dim 32c + 8g + j.
    if constexpr (TAGGED) stage_tagged<HD, NT>(a, kvh, sm_tq, sm_tk, sm_tv);
    h8_t qop[NC];
    {
        const int h = col & 7;
        const bool live = h < G;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float qv[8];
            if constexpr (TAGGED) {
                const float* qh = sm_tq + (live ? h : 0) * HD + 32 * c + 8 * g;
#pragma unroll
                for (int j = 0; j < 8; ++j) qv[j] = qh[j];
            } else {
                const float* qh = qg + (size_t)(live ? h : 0) * HD;
                const f4_t q0 = *reinterpret_cast<const f4_t*>(qh + 32 * c + 8 * g);
                const f4_t q1 = *reinterpret_cast<const f4_t*>(qh + 32 * c + 8 * g + 4);
                qv[0] = q0.x, qv[1] = q0.y, qv[2] = q0.z, qv[3] = q0.w;
                qv[4] = q1.x, qv[5] = q1.y, qv[6] = q1.z, qv[7] = q1.w;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = qv[j] * a.qscale;
                const _Float16 hi = (_Float16)v;
                const _Float16 lo = (_Float16)(v - (float)hi);
                qop[c][j] = !live ? (_Float16)0.0f : (col < 8 ? hi : lo);
            }
        }
    }

    // Running softmax state in the log2 domain. m_ref only moves when a block's
    // maximum exceeds it by more than LAZY (p stays <= 2^LAZY), so the O rows
    // are rescaled rarely instead of on every block.
    constexpr float LAZY = 8.0f;
    float m_ref = -INFINITY, l_run = 0.0f;
    f4_t o[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (; b < nblocks; b += step) {
        const int key0 = b * BLK;
        if constexpr (TAGGED) {
            if (b == (a.patch_pos >> 5)) patch_block<HD>(a, cur, sm_tk, sm_tv, lane);
        }
        // The next block's address (a page-table read for the paged cache) is
        // fetched before this block's math so its latency is hidden.
        typename KV::Addr next_addr{};
        if (b + step < nblocks) next_addr = src.addr(b + step);
        if constexpr (PREFETCH) {
            if (b + step < nblocks) src.load(nxt, next_addr, lane);
        }

        // ---- scores (log2 domain): lane group g, slot j = 4t + i (tile t,
        // row 4g + i) is key key0 + KV::key(g, j)
        float s[8];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NC; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[t][c], qop[c], acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) s[4 * t + i] = acc[i];
        }
        const bool tail = key0 + BLK > n || key0 < lo;
        const int nvalid = n - key0;  // keys of this block inside [lo, n) are
        const int nskip = lo - key0;  // the slots in [nskip, nvalid)
        float mb = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s[j] += mxd::dpp_f32<0x128>(s[j]);  // row_ror:8 = column h + 8: hi + lo
            if (tail) s[j] = KV::key(g, j) < nvalid && KV::key(g, j) >= nskip ? s[j] : -INFINITY;
            mb = fmaxf(mb, s[j]);
        }
        mb = fmaxf(mb, __shfl_xor(mb, 16));
        mb = fmaxf(mb, __shfl_xor(mb, 32));
        if (__any(mb > m_ref + LAZY)) {
            const float m_new = fmaxf(m_ref, mb);
            const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
            m_ref = m_new;
            l_run *= alpha;
            float ar[4];  // O row 4g+i is head slot (4g+i) mod 8 (hi or lo part)
#pragma unroll
            for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[d][i] *= ar[i];
        }

        h8_t pa;
        float psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = __builtin_amdgcn_exp2f(s[j] - m_ref);
            psum += p;
            const _Float16 hi = (_Float16)p;
            const _Float16 lo = (_Float16)(p - (float)hi);
            pa[j] = (col & 7) >= G ? (_Float16)0.0f : (col < 8 ? hi : lo);
        }
        l_run += psum;

        // ---- O += P.V; keys past n may hold stale bits (NaN/Inf): zero them.
        if (tail) {
            u4_t keep;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const int k0 = KV::key(g, 2 * w), k1 = KV::key(g, 2 * w + 1);
                keep[w] = (k0 < nvalid && k0 >= nskip ? 0x0000FFFFu : 0u) |
                          (k1 < nvalid && k1 >= nskip ? 0xFFFF0000u : 0u);
            }
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                u4_t v;
                __builtin_memcpy(&v, &cur.v[d], 16);
                v &= keep;
                __builtin_memcpy(&cur.v[d], &v, 16);
            }
        }
#pragma unroll
        for (int d = 0; d < ND; ++d) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, cur.v[d], o[d], 0, 0, 0);

        if constexpr (PREFETCH) {
            cur = nxt;
        } else if (b + step < nblocks) {
            src.load(cur, next_addr, lane);
        }
    }

    // ---- per-wave results: l summed over the 4 lane groups; all 16 O rows
    // (hi and lo parts) go to LDS unmasked. Folding hi + lo here with
    // cross-lane shuffles behind per-row branches serialised into one LDS round
    // trip per row (~2.5 us at head_dim 256).
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (lane < G) {
        sm_m[wave][lane] = m_ref;
        sm_l[wave][lane] = l_run;
    }
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm_o[wave][4 * g + i][16 * d + col] = o[d][i];
    __syncthreads();

    // ---- merge the waves (and write the partial or the output). First the
    // per-(wave, head) weights 2^(m_w - M) (over the total sum for a direct
    // output), then each value is row h (hi) + row h + 8 (lo) of every wave,
    // weighted.
    if (threadIdx.x < G) {
        const int h = threadIdx.x;
        float M = sm_m[0][h];
#pragma unroll
        for (int w = 1; w < W; ++w) M = fmaxf(M, sm_m[w][h]);
        float f[W], sl = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            f[w] = __builtin_amdgcn_exp2f(sm_m[w][h] - M);
            sl += f[w] * sm_l[w][h];
        }
        const float norm = out.direct ? 1.0f / sl : 1.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) sm_c[w][h] = f[w] * norm;
        if (!out.direct) {
            if constexpr (TAGGED) {
                mxd::tag_put(out.tml + 2 * h + 0, a.tag, M);
                mxd::tag_put(out.tml + 2 * h + 1, a.tag, sl);
            } else {
                out.pml[2 * h + 0] = M;
                out.pml[2 * h + 1] = sl;
            }
        }
    }
    __syncthreads();
    float* dst = out.direct ? out.orow : out.po;
    for (int idx = threadIdx.x; idx < G * HD; idx += NT) {
        const int h = idx / HD, dim = idx - h * HD;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) v += sm_c[w][h] * (sm_o[w][h][dim] + sm_o[w][h + 8][dim]);
        if constexpr (TAGGED)
            mxd::tag_put(out.trow + idx, a.tag, v);
        else if (out.direct && out.orow_h)
            out.orow_h[idx] = mxd::f2h_bits(v);
        else
            dst[idx] = v;
    }
    __syncthreads();  // the LDS rows are free for the next run
}

}  // namespace
