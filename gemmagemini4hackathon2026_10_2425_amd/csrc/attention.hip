// Single-query (decode) attention over a contiguous fp16 KV cache, split over
// the key axis (flash-decoding) and run on the matrix cores.
//
// Reference semantics (KL/kernels.metal:235-305): scores = scale * q . k_j in
// fp32, max-subtracted softmax in fp32, out = sum_j p_j v_j / sum_j p_j, GQA
// head mapping kvh = h / (n_heads / n_kv_heads). The reference keeps every
// score in threadgroup memory (context capped at 4096) and re-reads K/V once
// per query head; here:
//
//  * grid = (key splits, kv heads); a workgroup of 4 waves owns one kv head and
//    one split; each wave walks 32-key blocks of the split with an online
//    (running max / running sum) softmax in fp32.
//  * the G = n_heads / n_kv_heads query heads of the group ride in the columns
//    of one 16x16x32 fp16 MFMA, so each K and V element is loaded once for all
//    of them: S^T[key][col] = K[key][:] . Q^T[:][col].
//  * fp32 accuracy from fp16 matrix cores: q is split into hi = fp16(q) and
//    lo = fp16(q - hi) in columns h and h + 8 (G <= 8); the score of head h is
//    the sum of the two columns (products of fp16 values are exact in fp32),
//    one DPP row rotation away.
//    P is split the same way for the P.V product, so out keeps ~22 bits.
//  * the S^T accumulator layout (lane = column, 4 rows per lane group) is
//    already the A-operand layout of the P.V MFMA once the key rows are
//    permuted at load time, so P never leaves registers.
//  * K and V are cached in tiles of 32 positions stored in MFMA operand order,
//    so each operand is one fully coalesced 1 KiB wave load (every 16-lane
//    quarter-wave reads 256 contiguous bytes) and a block is one contiguous
//    8 KiB (hd 128) run per cache.
//  * 32-key blocks are dealt round-robin to the splits of a kv head (split s
//    takes blocks s, s+S, ...), so the grid streams the cache front to back;
//    each wave keeps one block in flight (prefetching the next one is a
//    tunable, measured slower).
//  * splits write unnormalised (O, max, sum) partials, merged by a second small
//    kernel with the log-sum-exp rule; a single split writes the output
//    directly. (A merge by the last-arriving split needs device-scope fences
//    in every workgroup, which on a multi-XCD part costs more than a launch.)
//  * the paged variant (a ragged batch of sequences over a pool of 16-key
//    pages) runs the same core: a 32-key block is two pages, each page holds
//    one half of a contiguous tile, and each lane addresses its own page, so
//    every operand is two 512-byte runs. Its default schedule deals the
//    batch's (sequence, kv head, block) items evenly over the workgroups that
//    fit the GPU at once, whatever the spread of lengths (measured on MI355X,
//    64 sequences of 128..8192 keys: 180 us against 251 us for a fixed number
//    of 16-block splits per sequence, which leaves the long ones for last);
//  * K and V are read with nontemporal loads: they stream through once.
#include "common.hpp"

#include <mutex>
#include <type_traits>
#include <vector>

#include "attn_core.hpp"
#include "internal.hpp"

namespace {

// Split `split` of S over the kv head's n keys (the last a.window of them
// under a sliding window): partials at split-major rows [split][n_heads] of
// ws_o / ws_ml, or the output directly when one split is active. An empty
// sequence writes a zero output.
template <int HD, int W, bool PF, typename KV>
__device__ __forceinline__ void attn_split(const AttnArgs& a, const KV& src, int n, int S, int split, int kvh,
                                           const float* qrow, float* orow, float* ws_o, float* ws_ml,
                                           uint16_t* orow_h = nullptr) {
    const int nblocks = (n + BLK - 1) / BLK;
    const int lo = window_lo(a, n), blo = lo / BLK;
    const size_t g0 = (size_t)kvh * a.G;
    if (nblocks == 0) {
        if (split == 0 && a.partials_only) {  // a zero output as a partial: O = 0, (max, sum) = (0, 1)
            for (int idx = threadIdx.x; idx < a.G * HD; idx += W * 64) ws_o[g0 * HD + idx] = 0.0f;
            for (int idx = threadIdx.x; idx < a.G; idx += W * 64) {
                ws_ml[(g0 + idx) * 2] = 0.0f;
                ws_ml[(g0 + idx) * 2 + 1] = 1.0f;
            }
        } else if (split == 0) {
            for (int idx = threadIdx.x; idx < a.G * HD; idx += W * 64) {
                if (orow_h)
                    orow_h[g0 * HD + idx] = 0;
                else
                    orow[g0 * HD + idx] = 0.0f;
            }
        }
        return;
    }
    const int n_active = min(S, nblocks - blo);
    if (split >= n_active) return;  // an empty split
    const size_t prow = (size_t)split * a.n_heads + g0;
    const CoreOut out{orow ? orow + g0 * HD : nullptr, ws_o + prow * HD, ws_ml + prow * 2,
                      n_active == 1 && !a.partials_only, nullptr, nullptr, orow_h ? orow_h + g0 * HD : nullptr};
    attn_core<HD, W, PF>(a, src, n, blo + split, S, nblocks, qrow + g0 * HD, out, 0, lo);
}

// Waves per SIMD the register allocation must allow. Left to itself the
// head_dim 256 core takes 224 VGPRs + 64 AGPRs, one wave per SIMD; capped at
// 256 registers (a spill of 7-9 dwords per lane) it runs two. The prefetch
// variant would spill 132 dwords and keeps its one wave. Measured on MI355X,
// two alternating runs: Gemma-4-E2B pp512 58.1-58.3k against 57.3-57.4k
// tok/s, Gemma-2B pp1024 122.0-122.2k against 120.6-121.6k; decode, whose
// head_dim 256 attention is 6 workgroups, unchanged.
template <int HD, bool PF>
constexpr int att_min_waves() {
    return HD == 256 && !PF ? 2 : 1;
}

template <int HD, int W, bool PF>
__global__ void __launch_bounds__(W * 64, (att_min_waves<HD, PF>())) attn_split_kernel(AttnArgs a) {
    const int kvh = blockIdx.y;
    const ContigKV<HD> src{a.k + (size_t)kvh * a.max_ctx * HD, a.v + (size_t)kvh * a.max_ctx * HD};
    const int n = n_keys_of(a);
    attn_split<HD, W, PF>(a, src, n, active_splits(a, attended_blocks(a, n)), blockIdx.x, kvh, a.q, a.out, a.ws_o,
                          a.ws_ml);
}

// Prefill: `rows` queries at positions pos0 .. pos0 + rows - 1 over the
// contiguous cache (their keys and values already appended); query t sees
// keys [0, pos0 + t] (a.n_keys = pos0 + 1). Grid (rows, n_kv): one workgroup
// per (query, kv head), one split, so each writes its output rows directly;
// the kv head's G query heads share every K/V tile as in decode. Workgroups
// start with the last (longest) rows, so the short ones fill the tail
// (Gemma-2B pp1024 on MI355X: 124.5-124.8k against 122.6-123.2k tok/s).
template <int HD, int W, bool PF>
__global__ void __launch_bounds__(W * 64, (att_min_waves<HD, PF>())) attn_prefill_kernel(AttnArgs a) {
    const int t = gridDim.x - 1 - blockIdx.x, kvh = blockIdx.y;
    const ContigKV<HD> src{a.k + (size_t)kvh * a.max_ctx * HD, a.v + (size_t)kvh * a.max_ctx * HD};
    const int n = min(a.n_keys + t, a.max_ctx);
    attn_split<HD, W, PF>(a, src, n, 1, 0, kvh, a.q + (size_t)t * a.q_stride,
                          a.out ? a.out + (size_t)t * a.out_stride : nullptr, a.ws_o, a.ws_ml,
                          a.out_h ? a.out_h + (size_t)t * a.out_stride : nullptr);
}

// Keys and splits of paged sequence seq (clamped so a bad length can never
// address past its page-table row).
__device__ __forceinline__ int paged_keys(const AttnArgs& a, int seq) {
    return max(0, min(a.seq_lens[seq], a.max_pages * mxd::PAGE_KEYS));
}
__device__ __forceinline__ int paged_splits(const AttnArgs& a, int n) {
    const int nblocks = (n + BLK - 1) / BLK;
    return min(a.n_splits, max(1, (nblocks + a.bps - 1) / a.bps));
}

template <int HD, int W, bool PF>
__global__ void __launch_bounds__(W * 64) attn_paged_kernel(AttnArgs a) {
    const int kvh = blockIdx.y, seq = blockIdx.z;
    const int n = paged_keys(a, seq);
    const PagedKV<HD> src{a.k, a.v, a.page_table + (size_t)seq * a.max_pages, (n + mxd::PAGE_KEYS - 1) / mxd::PAGE_KEYS,
                          a.n_pages, (size_t)a.n_kv * mxd::PAGE_KEYS * HD, kvh};
    const size_t ws_rows = (size_t)seq * a.n_splits * a.n_heads;
    attn_split<HD, W, PF>(a, src, n, paged_splits(a, n), blockIdx.x, kvh, a.q + (size_t)seq * a.q_stride,
                          a.out + (size_t)seq * a.out_stride, a.ws_o + ws_rows * HD, a.ws_ml + ws_rows * 2);
}

// ---------------------------------------------------------------------------
// Paged attention with a balanced schedule. The work is the list of every
// (sequence, kv head, 32-key block), ordered by sequence, then kv head, then
// block: sequence s contributes n_kv segments of nb(s) blocks. Workgroup w of
// NW takes items [w*T/NW, (w+1)*T/NW) of the T items, so every workgroup
// streams the same number of blocks whatever the spread of lengths. The range
// of a workgroup cuts the segments into pieces; a segment inside one range is
// written out directly, any other leaves one partial per piece, at slot w + sg
// (sg = the segment's index; along the monotone path of (workgroup, segment)
// pieces that sum strictly increases, so slots never collide, and there are
// at most NW + n_seqs * n_kv of them).
// ---------------------------------------------------------------------------

// Exclusive prefix of per-sequence blocks into pre[0..n_seqs]; returns the
// total. Every thread of the workgroup calls it.
template <int NT>
__device__ __forceinline__ int sk_block_prefix(const AttnArgs& a, int* pre) {
    __shared__ int wsum[NT / 64];
    const int ns = a.n_seqs;
    const int per = (ns + NT - 1) / NT;
    const int s0 = min(ns, (int)threadIdx.x * per), s1 = min(ns, s0 + per);
    int local = 0;
    for (int s = s0; s < s1; ++s) {
        const int nb = (paged_keys(a, s) + BLK - 1) / BLK;
        pre[s + 1] = nb;  // lengths first, turned into a prefix below
        local += nb;
    }
    // inclusive scan of the per-thread sums across the wave, then the waves
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = local;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(inc, d);
        if (lane >= d) inc += v;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        base += w < wave ? wsum[w] : 0;
        total += wsum[w];
    }
    // each thread rewrites only its own entries pre[s0+1 .. s1] (length ->
    // inclusive prefix), so no entry is read after another thread wrote it
    int run = base + inc - local;
    for (int s = s0; s < s1; ++s) {
        run += pre[s + 1];
        pre[s + 1] = run;
    }
    if (threadIdx.x == 0) pre[0] = 0;
    __syncthreads();
    return total;
}

// Workgroups that get work: enough that each streams at least SK_MIN_BLOCKS.
__device__ __forceinline__ int sk_active(long long T, int nw) {
    return (int)max(1LL, min((long long)nw, (T + SK_MIN_BLOCKS - 1) / SK_MIN_BLOCKS));
}

// The workgroup whose range holds item x (ranges are never empty: T >= nw).
__device__ __forceinline__ int sk_owner(long long x, long long T, int nw) {
    return (int)(((x + 1) * nw - 1) / T);
}

template <int HD, int W, bool PF>
__global__ void __launch_bounds__(W * 64) attn_paged_sk_kernel(AttnArgs a) {
    __shared__ int pre[SK_MAX_SEQS + 1];
    const int total = sk_block_prefix<W * 64>(a, pre);
    const int ns = a.n_seqs, nkv = a.n_kv;
    if (blockIdx.x == 0)
        for (int s = threadIdx.x; s <= ns; s += W * 64) a.sk_pre[s] = pre[s];
    const long long T = (long long)nkv * total;
    if (T == 0) return;
    const int nw = sk_active(T, a.sk_wgs);
    const int w = blockIdx.x;
    if (w >= nw) return;
    long long pos = (long long)w * T / nw;
    const long long end = (long long)(w + 1) * T / nw;

    // the sequence holding pos: the last s with nkv * pre[s] <= pos
    int lo = 0, hi = ns - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((long long)nkv * pre[mid] <= pos) lo = mid;
        else hi = mid - 1;
    }
    int seq = lo;
    const size_t page_stride = (size_t)nkv * mxd::PAGE_KEYS * HD;
    while (pos < end) {
        while ((long long)nkv * pre[seq + 1] <= pos) ++seq;  // skip finished and empty sequences
        const int nb = pre[seq + 1] - pre[seq];
        const long long base = (long long)nkv * pre[seq];
        const int kvh = (int)((pos - base) / nb);
        const long long seg0 = base + (long long)kvh * nb;
        const int b0 = (int)(pos - seg0);
        const int b1 = (int)min((long long)nb, end - seg0);
        const int n = paged_keys(a, seq);
        const PagedKV<HD> src{a.k, a.v, a.page_table + (size_t)seq * a.max_pages,
                              (n + mxd::PAGE_KEYS - 1) / mxd::PAGE_KEYS, a.n_pages, page_stride, kvh};
        const size_t g0 = (size_t)kvh * a.G;
        const size_t slot = (size_t)w + (size_t)seq * nkv + kvh;
        const CoreOut out{a.out + (size_t)seq * a.out_stride + g0 * HD, a.ws_o + slot * a.G * HD,
                          a.ws_ml + slot * a.G * 2, b0 == 0 && b1 == nb};
        attn_core<HD, W, PF>(a, src, n, b0, 1, b1, a.q + (size_t)seq * a.q_stride + g0 * HD, out);
        pos = seg0 + b1;
    }
}

// Merge of the balanced schedule: one thread per (sequence, head, dim). A
// segment inside one workgroup's range was written directly; an empty one
// gets zeros; any other sums its pieces (slots w + sg for its workgroups
// w0..w1) with the log-sum-exp rule.
constexpr int SKM_T = 128;

template <int HD>
__global__ void __launch_bounds__(SKM_T) attn_paged_sk_merge_kernel(AttnArgs a) {
    const int seq = blockIdx.y;
    const int idx = blockIdx.x * SKM_T + threadIdx.x;  // head * HD + dim
    if (idx >= a.n_heads * HD) return;
    const int head = idx / HD, dim = idx - head * HD;
    const int kvh = head / a.G, h = head - kvh * a.G;
    const int p0 = a.sk_pre[seq], p1 = a.sk_pre[seq + 1], tot = a.sk_pre[a.n_seqs];
    float* o = a.out + (size_t)seq * a.out_stride + idx;
    const int nb = p1 - p0;
    if (nb == 0) {
        *o = 0.0f;
        return;
    }
    const long long T = (long long)a.n_kv * tot;
    const int nw = sk_active(T, a.sk_wgs);
    const long long s0 = (long long)a.n_kv * p0 + (long long)kvh * nb;
    const int w0 = sk_owner(s0, T, nw), w1 = sk_owner(s0 + nb - 1, T, nw);
    if (w0 == w1) return;
    const size_t slot0 = (size_t)w0 + (size_t)seq * a.n_kv + kvh;
    const float* pml = a.ws_ml + (slot0 * a.G + h) * 2;
    const float* po = a.ws_o + (slot0 * a.G + h) * HD + dim;
    const size_t sml = (size_t)a.G * 2, so = (size_t)a.G * HD;
    const int np = w1 - w0 + 1;
    float M = -INFINITY;
    for (int i = 0; i < np; ++i) M = fmaxf(M, pml[i * sml]);
    float num = 0.0f, den = 0.0f;
    for (int i = 0; i < np; ++i) {
        const float f = exp2f(pml[i * sml] - M);
        num += f * po[i * so];
        den += f * pml[i * sml + 1];
    }
    *o = num / den;
}

// out[h] = sum_s 2^(M_s - M) O_s / sum_s 2^(M_s - M) L_s over the active
// splits (log-sum-exp rule). A workgroup of MG_T = 256 threads merges MG_D = 32
// dims of one query head: thread (grp, d) sums its dim over splits grp,
// grp + MG, ...; its first PRE partials are loaded before the (M_s, L_s) pass
// so the two latencies overlap, which makes the common case (up to MG * PRE =
// 96 splits, the long-context default) one round trip. The groups are combined in LDS in a fixed order
// (deterministic).
constexpr int MG_D = 32;
constexpr int MG = 8;
constexpr int MG_T = MG * MG_D;
constexpr int PRE = 12;

template <int HD>
__device__ __forceinline__ void attn_merge_core(const AttnArgs& a, int n_active, int head, int dchunk, float* orow,
                                                const float* ws_o, const float* ws_ml) {
    __shared__ float sw[MAX_SPLITS];
    __shared__ float sl[MAX_SPLITS];
    __shared__ float red[2][MG_T / 64];
    __shared__ float part[MG - 1][MG_D];
    if (n_active <= 1) return;
    const int tid = threadIdx.x;
    const int grp = tid / MG_D, dim = dchunk * MG_D + (tid - grp * MG_D);
    const float* po = ws_o + (size_t)head * HD + dim;
    const size_t stride = (size_t)a.n_heads * HD;

    float pre[PRE];
#pragma unroll
    for (int u = 0; u < PRE; ++u) {
        const int sp = grp + MG * u;
        pre[u] = sp < n_active ? po[(size_t)sp * stride] : 0.0f;
    }
    float mloc = -INFINITY;
    for (int sp = tid; sp < n_active; sp += MG_T) {
        const float m = ws_ml[((size_t)sp * a.n_heads + head) * 2];
        sw[sp] = m;
        sl[sp] = ws_ml[((size_t)sp * a.n_heads + head) * 2 + 1];
        mloc = fmaxf(mloc, m);
    }
    mloc = mxd::wave_max(mloc);
    if ((tid & 63) == 0) red[0][tid >> 6] = mloc;
    __syncthreads();
    float M = red[0][0];
#pragma unroll
    for (int w = 1; w < MG_T / 64; ++w) M = fmaxf(M, red[0][w]);
    float lloc = 0.0f;
    for (int sp = tid; sp < n_active; sp += MG_T) {
        const float f = exp2f(sw[sp] - M);
        sw[sp] = f;
        lloc += f * sl[sp];
    }
    lloc = mxd::wave_sum(lloc);
    if ((tid & 63) == 0) red[1][tid >> 6] = lloc;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < MG_T / 64; ++w) L += red[1][w];

    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < PRE; ++u) {
        const int sp = grp + MG * u;
        if (sp < n_active) acc += sw[sp] * pre[u];
    }
    // More than MG * PRE splits (long contexts over few kv heads): the rest,
    // four loads in flight at a time.
    int sp = grp + MG * PRE;
    for (; sp + 3 * MG < n_active; sp += 4 * MG) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = po[(size_t)(sp + MG * u) * stride];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += sw[sp + MG * u] * v[u];
    }
    for (; sp < n_active; sp += MG) acc += sw[sp] * po[(size_t)sp * stride];
    if (grp > 0) part[grp - 1][dim - dchunk * MG_D] = acc;
    __syncthreads();
    if (grp == 0) {
        float tot = acc;
#pragma unroll
        for (int g2 = 0; g2 < MG - 1; ++g2) tot += part[g2][dim - dchunk * MG_D];
        orow[(size_t)head * HD + dim] = tot / L;
    }
}

// Grid (n_heads * HD / MG_D): workgroup x merges dims (x % (HD/MG_D)) * MG_D ..
// of head x / (HD/MG_D).
template <int HD>
__global__ void __launch_bounds__(MG_T) attn_merge_kernel(AttnArgs a) {
    const int nblocks = attended_blocks(a, n_keys_of(a));
    const int n_active = min(active_splits(a, nblocks), nblocks);
    constexpr int NCH = HD / MG_D;
    attn_merge_core<HD>(a, n_active, blockIdx.x / NCH, blockIdx.x % NCH, a.out, a.ws_o, a.ws_ml);
}

template <int HD>
__global__ void __launch_bounds__(MG_T) attn_paged_merge_kernel(AttnArgs a) {
    const int seq = blockIdx.y;
    const int n = paged_keys(a, seq);
    const int n_active = min(paged_splits(a, n), (n + BLK - 1) / BLK);
    const size_t ws_rows = (size_t)seq * a.n_splits * a.n_heads;
    constexpr int NCH = HD / MG_D;
    attn_merge_core<HD>(a, n_active, blockIdx.x / NCH, blockIdx.x % NCH, a.out + (size_t)seq * a.out_stride,
                        a.ws_o + ws_rows * HD,
                        a.ws_ml + ws_rows * 2);
}

// Waves per workgroup (ATT_W: 4 or 8) and whether each wave prefetches its
// next block (ATT_PF = 1; off by default: measured on MI355X, one block in
// flight per wave with nontemporal loads streams faster, 29.5 vs 31.0 us at
// L = 32768 and 230 vs 265 us on the 64-sequence paged batch).
int att_waves() { return mxd::tunable("ATT_W", ATT_WAVES) == 8 ? 8 : 4; }
bool att_prefetch(int hd) { (void)hd; return mxd::tunable("ATT_PF", 2) == 1; }

// Waves per workgroup at head_dim hd: head_dim 512 always takes 4 (its
// per-wave O rows fill 129 KiB of LDS at 4 waves).
int waves_for(int hd) { return hd >= 512 ? 4 : att_waves(); }

template <int HD>
void launch_split(const dim3& grid, hipStream_t s, const AttnArgs& a) {
    const int w = waves_for(HD);
    const bool pf = att_prefetch(HD);
    if constexpr (HD >= 512) {
        if (pf) hipLaunchKernelGGL((attn_split_kernel<HD, 4, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((attn_split_kernel<HD, 4, false>), grid, dim3(256), 0, s, a);
    } else if (w == 8) {
        if (pf) hipLaunchKernelGGL((attn_split_kernel<HD, 8, true>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((attn_split_kernel<HD, 8, false>), grid, dim3(512), 0, s, a);
    } else {
        if (pf) hipLaunchKernelGGL((attn_split_kernel<HD, 4, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((attn_split_kernel<HD, 4, false>), grid, dim3(256), 0, s, a);
    }
}

template <int HD>
void launch_paged(const dim3& grid, hipStream_t s, const AttnArgs& a) {
    const int w = att_waves();
    const bool pf = att_prefetch(HD);
    if (w == 8) {
        if (pf) hipLaunchKernelGGL((attn_paged_kernel<HD, 8, true>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((attn_paged_kernel<HD, 8, false>), grid, dim3(512), 0, s, a);
    } else {
        if (pf) hipLaunchKernelGGL((attn_paged_kernel<HD, 4, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((attn_paged_kernel<HD, 4, false>), grid, dim3(256), 0, s, a);
    }
}

template <int HD>
void launch_paged_sk(int nw, hipStream_t s, const AttnArgs& a) {
    const int w = att_waves();
    const bool pf = att_prefetch(HD);
    if (w == 8) {
        if (pf) hipLaunchKernelGGL((attn_paged_sk_kernel<HD, 8, true>), dim3(nw), dim3(512), 0, s, a);
        else hipLaunchKernelGGL((attn_paged_sk_kernel<HD, 8, false>), dim3(nw), dim3(512), 0, s, a);
    } else {
        if (pf) hipLaunchKernelGGL((attn_paged_sk_kernel<HD, 4, true>), dim3(nw), dim3(256), 0, s, a);
        else hipLaunchKernelGGL((attn_paged_sk_kernel<HD, 4, false>), dim3(nw), dim3(256), 0, s, a);
    }
}

// Splits per kv head: about ATT_WGCU (default 3, as many as stay resident at
// head_dim 128) workgroups per CU over the whole grid, and never more splits
// than 32-key blocks.
int target_splits(int n_kv) {
    const int per_cu = max(1, min(16, mxd::tunable("ATT_WGCU", 3)));
    return min(MAX_SPLITS, (per_cu * 256 + n_kv - 1) / n_kv);
}

// Up to 4 blocks per wave take one split, which writes the output without a
// merge launch (measured: a second launch costs more than the serial blocks
// it saves). Longer contexts take enough splits that every wave has at most
// one block, capped by the occupancy target. active_splits is the same rule
// on the device.
int single_blocks(int hd) { return mxd::tunable("ATT_SINGLE", 4 * waves_for(hd)); }
int splits_for(int max_keys, int n_kv, int hd) {
    const int nblocks = (max_keys + BLK - 1) / BLK;
    const int w = waves_for(hd);
    if (nblocks <= single_blocks(hd)) return 1;
    const int one_per_wave = (nblocks + w - 1) / w;
    return max(1, min(one_per_wave, target_splits(n_kv)));
}

// Blocks a query attends to at most: a sliding window of `window` keys starts
// anywhere inside a block, so it spans up to (window + 31) / 32 + 1 of them.
int max_keys_attended(int max_keys, int window) {
    return window > 0 ? min(max_keys, window + BLK) : max_keys;
}

// Calls f with std::integral_constant<int, HD> for the supported head dims
// (64: Llama-3.2-1B; 128: Llama-3-8B; 256: Gemma-2B and Gemma-4's sliding
// layers; with WIDE also 512: Gemma-4's full layers); the callers have
// checked head_dim.
template <bool WIDE = false, typename F>
void with_head_dim(int head_dim, F&& f) {
    if (head_dim == 64) f(std::integral_constant<int, 64>{});
    else if (head_dim == 128) f(std::integral_constant<int, 128>{});
    else if constexpr (WIDE) {
        if (head_dim == 512) f(std::integral_constant<int, 512>{});
        else f(std::integral_constant<int, 256>{});
    } else {
        f(std::integral_constant<int, 256>{});
    }
}

}  // namespace

extern "C" size_t mxd_attention_workspace_size(int n_heads, int n_kv_heads, int head_dim, int max_ctx) {
    (void)max_ctx;
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) return 0;
    const size_t splits = (size_t)target_splits(n_kv_heads);
    return splits * n_heads * (head_dim + 2) * sizeof(float);
}

namespace {

// mxd_attention / mxd_attention_window.
int attention_impl(const char* name, const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                   int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys, const int32_t* pos_dev,
                   int window, float scale, void* workspace, size_t ws_bytes, mxd_stream_t stream) {
    MXD_REQUIRE(q && kcache && vcache && out, MXD_ERR_INVALID_ARG, "%s: null pointer", name);
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, MXD_ERR_INVALID_ARG,
                "%s: n_heads=%d must be a positive multiple of n_kv_heads=%d", name, n_heads, n_kv_heads);
    const int G = n_heads / n_kv_heads;
    MXD_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, MXD_ERR_UNSUPPORTED,
                "%s: group size %d (n_heads / n_kv_heads) must be 1, 2, 4 or 8", name, G);
    MXD_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512, MXD_ERR_UNSUPPORTED,
                "%s: head_dim %d (64, 128, 256 or 512)", name, head_dim);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED,
                "%s: max_ctx=%d must be a positive multiple of 32", name, max_ctx);
    MXD_REQUIRE(pos_dev || (n_keys >= 1 && n_keys <= max_ctx), MXD_ERR_INVALID_ARG,
                "%s: n_keys=%d outside [1, max_ctx=%d]", name, n_keys, max_ctx);
    MXD_REQUIRE(window >= 0, MXD_ERR_INVALID_ARG, "%s: window=%d", name, window);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kcache) |
                         reinterpret_cast<uintptr_t>(vcache);
    MXD_REQUIRE((al & 15) == 0, MXD_ERR_UNSUPPORTED, "%s: q, kcache, vcache must be 16-byte aligned", name);

    const int n_splits = splits_for(max_keys_attended(pos_dev ? max_ctx : n_keys, window), n_kv_heads, head_dim);
    const size_t need = (size_t)n_splits * n_heads * (head_dim + 2) * sizeof(float);
    MXD_REQUIRE(n_splits == 1 || (workspace && ws_bytes >= need), MXD_ERR_WORKSPACE,
                "%s: workspace of %zu bytes needed (got %zu)", name, need, ws_bytes);
    MXD_REQUIRE(!workspace || (reinterpret_cast<uintptr_t>(workspace) & 15) == 0, MXD_ERR_UNSUPPORTED,
                "%s: workspace must be 16-byte aligned", name);

    AttnArgs a;
    a.q = q;
    a.k = kcache;
    a.v = vcache;
    a.out = out;
    // Workspace: [O partials | (max, sum) partials]
    a.ws_o = static_cast<float*>(workspace);
    a.ws_ml = workspace ? a.ws_o + (size_t)n_splits * n_heads * head_dim : nullptr;
    a.pos_dev = pos_dev;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.G = G;
    a.max_ctx = max_ctx;
    a.n_keys = n_keys;
    a.n_splits = n_splits;
    a.qscale = scale * LOG2E;
    a.auto_splits = true;
    a.single_blocks = single_blocks(head_dim);
    a.waves = waves_for(head_dim);
    a.window = window;

    hipStream_t s = mxd::as_stream(stream);
    const dim3 grid(n_splits, n_kv_heads);
    with_head_dim<true>(head_dim, [&](auto hd) {
        constexpr int HD = decltype(hd)::value;
        launch_split<HD>(grid, s, a);
        if (n_splits > 1) hipLaunchKernelGGL(attn_merge_kernel<HD>, dim3(n_heads * HD / MG_D), dim3(MG_T), 0, s, a);
    });
    return mxd::check_launch(name);
}

}  // namespace

extern "C" int mxd_attention(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out, int n_heads,
                             int n_kv_heads, int head_dim, int max_ctx, int n_keys, const int32_t* pos_dev,
                             float scale, void* workspace, size_t ws_bytes, mxd_stream_t stream) {
    return attention_impl("mxd_attention", q, kcache, vcache, out, n_heads, n_kv_heads, head_dim, max_ctx, n_keys,
                          pos_dev, 0, scale, workspace, ws_bytes, stream);
}

extern "C" int mxd_attention_window(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                                    int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys,
                                    const int32_t* pos_dev, int window, float scale, void* workspace,
                                    size_t ws_bytes, mxd_stream_t stream) {
    return attention_impl("mxd_attention_window", q, kcache, vcache, out, n_heads, n_kv_heads, head_dim, max_ctx,
                          n_keys, pos_dev, window, scale, workspace, ws_bytes, stream);
}

extern "C" int mxd_attention_split(const float* q, const uint16_t* kcache, const uint16_t* vcache, int n_heads,
                                   int n_kv_heads, int head_dim, int max_ctx, int n_keys, const int32_t* pos_dev,
                                   float scale, int n_splits, float* partials, size_t partial_bytes,
                                   mxd_stream_t stream) {
    return mxd_attention_split_window(q, kcache, vcache, n_heads, n_kv_heads, head_dim, max_ctx, n_keys, pos_dev, 0,
                                      scale, n_splits, partials, partial_bytes, stream);
}

extern "C" int mxd_attention_split_window(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                                          int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys,
                                          const int32_t* pos_dev, int window, float scale, int n_splits,
                                          float* partials, size_t partial_bytes, mxd_stream_t stream) {
    MXD_REQUIRE(window >= 0, MXD_ERR_INVALID_ARG, "mxd_attention_split: window=%d", window);
    MXD_REQUIRE(q && kcache && vcache && partials, MXD_ERR_INVALID_ARG, "mxd_attention_split: null pointer");
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, MXD_ERR_INVALID_ARG,
                "mxd_attention_split: n_heads=%d must be a positive multiple of n_kv_heads=%d", n_heads, n_kv_heads);
    const int G = n_heads / n_kv_heads;
    MXD_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, MXD_ERR_UNSUPPORTED,
                "mxd_attention_split: group size %d (n_heads / n_kv_heads) must be 1, 2, 4 or 8", G);
    MXD_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512, MXD_ERR_UNSUPPORTED,
                "mxd_attention_split: head_dim %d (64, 128, 256 or 512)", head_dim);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_attention_split: max_ctx=%d must be a positive multiple of 32", max_ctx);
    MXD_REQUIRE(pos_dev || (n_keys >= 1 && n_keys <= max_ctx), MXD_ERR_INVALID_ARG,
                "mxd_attention_split: n_keys=%d outside [1, max_ctx=%d]", n_keys, max_ctx);
    MXD_REQUIRE(n_splits >= 1 && n_splits <= MAX_SPLITS, MXD_ERR_INVALID_ARG,
                "mxd_attention_split: n_splits=%d outside [1, %d]", n_splits, MAX_SPLITS);
    const size_t need = (size_t)n_splits * n_heads * (head_dim + 2) * sizeof(float);
    MXD_REQUIRE(partial_bytes >= need, MXD_ERR_WORKSPACE, "mxd_attention_split: %zu partial bytes needed (got %zu)",
                need, partial_bytes);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kcache) |
                         reinterpret_cast<uintptr_t>(vcache) | reinterpret_cast<uintptr_t>(partials);
    MXD_REQUIRE((al & 15) == 0, MXD_ERR_UNSUPPORTED,
                "mxd_attention_split: q, kcache, vcache, partials must be 16-byte aligned");
    AttnArgs a;
    a.q = q;
    a.k = kcache;
    a.v = vcache;
    a.out = nullptr;
    a.ws_o = partials;
    a.ws_ml = partials + (size_t)n_splits * n_heads * head_dim;
    a.pos_dev = pos_dev;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.G = G;
    a.max_ctx = max_ctx;
    a.n_keys = n_keys;
    a.n_splits = n_splits;
    a.qscale = scale * LOG2E;
    a.partials_only = true;
    a.window = window;
    hipStream_t s = mxd::as_stream(stream);
    const dim3 grid(n_splits, n_kv_heads);
    with_head_dim<true>(head_dim, [&](auto hd) { launch_split<decltype(hd)::value>(grid, s, a); });
    return mxd::check_launch("mxd_attention_split");
}

namespace {
// 32-key blocks per split of a paged sequence (ATT_BPS, 4..256).
int paged_bps() { return max(4, min(256, mxd::tunable("ATT_BPS", PAGED_BPS))); }
int paged_split_max(int max_keys) {
    const int nblocks = (max_keys + BLK - 1) / BLK;
    const int bps = paged_bps();
    return min(MAX_SPLITS, max(1, (nblocks + bps - 1) / bps));
}

// The balanced schedule serves batches of up to SK_MAX_SEQS sequences whose
// item count fits an int (ATT_SCHED = 2 selects per-sequence splits instead).
bool use_balanced(int n_seqs, int max_keys, int n_kv) {
    const long long items = (long long)n_seqs * ((max_keys + BLK - 1) / BLK) * n_kv;
    return mxd::tunable("ATT_SCHED", 1) != 2 && n_seqs <= SK_MAX_SEQS && items < (1LL << 31);
}

template <typename K>
int resident_wgs(K kernel, int threads) {
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess) per_cu = 1;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    return max(1, per_cu) * max(1, cus);
}

// Workgroups of the balanced schedule: ATT_SKWG per CU, by default as many as
// stay resident at once (one round, every workgroup with the same work).
template <int HD>
int sk_wgs_hd() {
    const int w = att_waves();
    const bool pf = att_prefetch(HD);
    int n;
    if (w == 8) n = pf ? resident_wgs(attn_paged_sk_kernel<HD, 8, true>, 512) : resident_wgs(attn_paged_sk_kernel<HD, 8, false>, 512);
    else n = pf ? resident_wgs(attn_paged_sk_kernel<HD, 4, true>, 256) : resident_wgs(attn_paged_sk_kernel<HD, 4, false>, 256);
    const int per_cu = mxd::tunable("ATT_SKWG", 0);
    if (per_cu > 0) {
        int dev = 0, cus = 256;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
        n = min(64, per_cu) * cus;
    }
    return n;
}
int sk_wgs(int hd) { return hd == 64 ? sk_wgs_hd<64>() : hd == 128 ? sk_wgs_hd<128>() : sk_wgs_hd<256>(); }

// Workspace of the balanced schedule: partial slots (O rows, then (max, sum)
// pairs) and the n_seqs + 1 block prefix.
size_t sk_slots(int nw, int n_seqs, int n_kv) { return (size_t)nw + (size_t)n_seqs * n_kv; }
size_t sk_workspace(int nw, int n_seqs, int n_heads, int n_kv, int hd) {
    const int G = n_heads / n_kv;
    return sk_slots(nw, n_seqs, n_kv) * G * (hd + 2) * sizeof(float) + ((size_t)n_seqs + 1) * sizeof(int32_t);
}
}  // namespace

namespace {

int attention_prefill_impl(const char* name, const float* q, int q_stride, const uint16_t* kcache,
                           const uint16_t* vcache, float* out, int out_stride, int n_heads, int n_kv_heads,
                           int head_dim, int max_ctx, int pos0, int rows, int window, float scale,
                           mxd_stream_t stream, uint16_t* out_h = nullptr) {
    MXD_REQUIRE(q && kcache && vcache && (out || out_h), MXD_ERR_INVALID_ARG, "%s: null pointer", name);
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, MXD_ERR_INVALID_ARG,
                "%s: n_heads=%d must be a positive multiple of n_kv_heads=%d", name, n_heads, n_kv_heads);
    const int G = n_heads / n_kv_heads;
    MXD_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, MXD_ERR_UNSUPPORTED,
                "%s: group size %d (n_heads / n_kv_heads) must be 1, 2, 4 or 8", name, G);
    MXD_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512, MXD_ERR_UNSUPPORTED,
                "%s: head_dim %d (64, 128, 256 or 512)", name, head_dim);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED,
                "%s: max_ctx=%d must be a positive multiple of 32", name, max_ctx);
    MXD_REQUIRE(rows >= 1 && pos0 >= 0 && (long long)pos0 + rows <= max_ctx, MXD_ERR_INVALID_ARG,
                "%s: positions [%d, %d + %d) outside [0, max_ctx=%d)", name, pos0, pos0, rows, max_ctx);
    MXD_REQUIRE(q_stride >= n_heads * head_dim && out_stride >= n_heads * head_dim && q_stride % 4 == 0,
                MXD_ERR_INVALID_ARG, "%s: q_stride=%d out_stride=%d below n_heads * head_dim = %d "
                "(q_stride a multiple of 4)", name, q_stride, out_stride, n_heads * head_dim);
    MXD_REQUIRE(window >= 0, MXD_ERR_INVALID_ARG, "%s: window=%d", name, window);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kcache) |
                         reinterpret_cast<uintptr_t>(vcache);
    MXD_REQUIRE((al & 15) == 0, MXD_ERR_UNSUPPORTED, "%s: q, kcache, vcache must be 16-byte aligned", name);
    AttnArgs a;
    a.q = q;
    a.k = kcache;
    a.v = vcache;
    a.out = out_h ? nullptr : out;
    a.out_h = out_h;
    a.ws_o = nullptr;
    a.ws_ml = nullptr;
    a.pos_dev = nullptr;
    a.q_stride = q_stride;
    a.out_stride = out_stride;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.G = G;
    a.max_ctx = max_ctx;
    a.n_keys = pos0 + 1;
    a.n_splits = 1;
    a.qscale = scale * LOG2E;
    a.window = window;
    hipStream_t s = mxd::as_stream(stream);
    const dim3 grid(rows, n_kv_heads);
    with_head_dim<true>(head_dim, [&](auto hd) {
        hipLaunchKernelGGL((attn_prefill_kernel<decltype(hd)::value, ATT_WAVES, false>), grid, dim3(ATT_WAVES * 64), 0,
                           s, a);
    });
    return mxd::check_launch(name);
}

}  // namespace

extern "C" int mxd_attention_prefill(const float* q, int q_stride, const uint16_t* kcache, const uint16_t* vcache,
                                     float* out, int out_stride, int n_heads, int n_kv_heads, int head_dim,
                                     int max_ctx, int pos0, int rows, float scale, mxd_stream_t stream) {
    return attention_prefill_impl("mxd_attention_prefill", q, q_stride, kcache, vcache, out, out_stride, n_heads,
                                  n_kv_heads, head_dim, max_ctx, pos0, rows, 0, scale, stream);
}

extern "C" int mxd_attention_prefill_window(const float* q, int q_stride, const uint16_t* kcache,
                                            const uint16_t* vcache, float* out, int out_stride, int n_heads,
                                            int n_kv_heads, int head_dim, int max_ctx, int pos0, int rows,
                                            int window, float scale, mxd_stream_t stream) {
    return attention_prefill_impl("mxd_attention_prefill_window", q, q_stride, kcache, vcache, out, out_stride,
                                  n_heads, n_kv_heads, head_dim, max_ctx, pos0, rows, window, scale, stream);
}

// mxd_attention_prefill_window with fp16 output rows (the engines' prefill,
// whose o projection takes the attention rows rounded to fp16).
int mxd::attention_prefill_h16(const float* q, int q_stride, const uint16_t* kcache, const uint16_t* vcache,
                               uint16_t* out, int out_stride, int n_heads, int n_kv_heads, int head_dim, int max_ctx,
                               int pos0, int rows, int window, float scale, hipStream_t stream) {
    return attention_prefill_impl("attention_prefill_h16", q, q_stride, kcache, vcache, nullptr, out_stride, n_heads,
                                  n_kv_heads, head_dim, max_ctx, pos0, rows, window, scale,
                                  reinterpret_cast<mxd_stream_t>(stream), out);
}

extern "C" size_t mxd_attention_paged_workspace_size(int n_heads, int n_kv_heads, int head_dim, int n_seqs,
                                                     int max_keys) {
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || n_seqs <= 0 || max_keys <= 0) return 0;
    if (n_heads % n_kv_heads == 0 && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
        use_balanced(n_seqs, max_keys, n_kv_heads))
        return sk_workspace(sk_wgs(head_dim), n_seqs, n_heads, n_kv_heads, head_dim);
    return (size_t)n_seqs * paged_split_max(max_keys) * n_heads * (head_dim + 2) * sizeof(float);
}

extern "C" int mxd_attention_paged(const float* q, int q_stride, const uint16_t* kpool, const uint16_t* vpool,
                                   int n_pages, const int32_t* page_table, int max_pages, const int32_t* seq_lens,
                                   int n_seqs, float* out, int out_stride, int n_heads, int n_kv_heads, int head_dim,
                                   int max_keys, float scale, void* workspace, size_t ws_bytes,
                                   mxd_stream_t stream) {
    MXD_REQUIRE(q && kpool && vpool && page_table && seq_lens && out, MXD_ERR_INVALID_ARG,
                "mxd_attention_paged: null pointer");
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, MXD_ERR_INVALID_ARG,
                "mxd_attention_paged: n_heads=%d must be a positive multiple of n_kv_heads=%d", n_heads, n_kv_heads);
    const int G = n_heads / n_kv_heads;
    MXD_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, MXD_ERR_UNSUPPORTED,
                "mxd_attention_paged: group size %d (n_heads / n_kv_heads) must be 1, 2, 4 or 8", G);
    MXD_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, MXD_ERR_UNSUPPORTED,
                "mxd_attention_paged: head_dim %d (64, 128 or 256)", head_dim);
    MXD_REQUIRE(n_pages > 0 && max_pages > 0 && n_seqs > 0 && n_seqs <= 65535, MXD_ERR_INVALID_ARG,
                "mxd_attention_paged: n_pages=%d max_pages=%d n_seqs=%d", n_pages, max_pages, n_seqs);
    MXD_REQUIRE(max_keys >= 1 && max_keys <= max_pages * mxd::PAGE_KEYS, MXD_ERR_INVALID_ARG,
                "mxd_attention_paged: max_keys=%d outside [1, max_pages*16=%d]", max_keys,
                max_pages * mxd::PAGE_KEYS);
    MXD_REQUIRE(q_stride >= n_heads * head_dim && out_stride >= n_heads * head_dim && q_stride % 4 == 0,
                MXD_ERR_INVALID_ARG, "mxd_attention_paged: q_stride=%d / out_stride=%d below n_heads*head_dim=%d "
                "(q_stride a multiple of 4)", q_stride, out_stride, n_heads * head_dim);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kpool) |
                         reinterpret_cast<uintptr_t>(vpool);
    MXD_REQUIRE((al & 15) == 0, MXD_ERR_UNSUPPORTED, "mxd_attention_paged: q, kpool, vpool must be 16-byte aligned");
    const bool balanced = use_balanced(n_seqs, max_keys, n_kv_heads);
    const int s_max = paged_split_max(max_keys);
    const int nw = balanced ? sk_wgs(head_dim) : 0;
    const size_t need = balanced ? sk_workspace(nw, n_seqs, n_heads, n_kv_heads, head_dim)
                                 : (size_t)n_seqs * s_max * n_heads * (head_dim + 2) * sizeof(float);
    MXD_REQUIRE((!balanced && s_max == 1) || (workspace && ws_bytes >= need), MXD_ERR_WORKSPACE,
                "mxd_attention_paged: workspace of %zu bytes needed (got %zu)", need, ws_bytes);
    MXD_REQUIRE(!workspace || (reinterpret_cast<uintptr_t>(workspace) & 15) == 0, MXD_ERR_UNSUPPORTED,
                "mxd_attention_paged: workspace must be 16-byte aligned");

    AttnArgs a;
    a.q = q;
    a.k = kpool;
    a.v = vpool;
    a.out = out;
    a.ws_o = static_cast<float*>(workspace);
    if (balanced) {
        const size_t slots = sk_slots(nw, n_seqs, n_kv_heads);
        a.ws_ml = a.ws_o + slots * G * head_dim;
        a.sk_pre = reinterpret_cast<int32_t*>(a.ws_ml + slots * G * 2);
    } else {
        a.ws_ml = workspace ? a.ws_o + (size_t)n_seqs * s_max * n_heads * head_dim : nullptr;
    }
    a.n_seqs = n_seqs;
    a.sk_wgs = nw;
    a.pos_dev = nullptr;
    a.page_table = page_table;
    a.seq_lens = seq_lens;
    a.max_pages = max_pages;
    a.n_pages = n_pages;
    a.q_stride = q_stride;
    a.out_stride = out_stride;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.G = G;
    a.max_ctx = max_pages * mxd::PAGE_KEYS;
    a.n_keys = 0;
    a.n_splits = s_max;
    a.bps = paged_bps();
    a.qscale = scale * LOG2E;

    hipStream_t s = mxd::as_stream(stream);
    if (balanced) {
        const dim3 mgrid((n_heads * head_dim + SKM_T - 1) / SKM_T, n_seqs);
        with_head_dim(head_dim, [&](auto hd) {
            constexpr int HD = decltype(hd)::value;
            launch_paged_sk<HD>(nw, s, a);
            hipLaunchKernelGGL(attn_paged_sk_merge_kernel<HD>, mgrid, dim3(SKM_T), 0, s, a);
        });
        return mxd::check_launch("mxd_attention_paged");
    }
    const dim3 grid(s_max, n_kv_heads, n_seqs);
    with_head_dim(head_dim, [&](auto hd) {
        constexpr int HD = decltype(hd)::value;
        launch_paged<HD>(grid, s, a);
        if (s_max > 1)
            hipLaunchKernelGGL(attn_paged_merge_kernel<HD>, dim3(n_heads * HD / MG_D, n_seqs), dim3(MG_T), 0, s, a);
    });
    return mxd::check_launch("mxd_attention_paged");
}

// ---------------------------------------------------------------------------
// mxd_attention without a workspace argument, for callers that cannot
// allocate: the split partials live in a file-scope device array, one per GPU,
// held until the process ends. Its device address comes from
// hipGetSymbolAddress on each device's first call (the host-side name of the
// array is not a device address) and is kept per device.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)8 << 20;  // 8 MiB per GPU
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_dev;  // scratch's address on device d, or null

int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return mxd::fail(MXD_ERR_HIP, "mxd_attention_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((size_t)dev >= g_scratch_dev.size()) g_scratch_dev.resize(dev + 1, nullptr);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return mxd::fail(MXD_ERR_HIP, "mxd_attention_noalloc: hipGetSymbolAddress(scratch): %s",
                             hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return MXD_OK;
}

}  // namespace

extern "C" size_t mxd_attention_noalloc_max_scratch(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int mxd_attention_noalloc(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                                     int n_heads, int n_kv_heads, int head_dim, int max_ctx, int n_keys,
                                     const int32_t* n_keys_dev, float scale, mxd_stream_t stream) {
    // The partials mxd_attention would take from its workspace; the shape
    // itself is checked there.
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && max_ctx > 0, MXD_ERR_INVALID_ARG,
                "mxd_attention_noalloc: n_heads=%d n_kv_heads=%d head_dim=%d max_ctx=%d", n_heads, n_kv_heads,
                head_dim, max_ctx);
    const int splits = splits_for(n_keys_dev ? max_ctx : max(n_keys, 1), n_kv_heads, head_dim);
    const size_t need = (size_t)splits * n_heads * (head_dim + 2) * sizeof(float);
    MXD_REQUIRE(need <= NOALLOC_SCRATCH_BYTES, MXD_ERR_UNSUPPORTED,
                "mxd_attention_noalloc: this shape needs %zu bytes of split partials, above the %zu-byte scratch",
                need, NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (int rc = scratch_address(&ws)) return rc;
    return mxd_attention(q, kcache, vcache, out, n_heads, n_kv_heads, head_dim, max_ctx, n_keys, n_keys_dev, scale,
                         ws, NOALLOC_SCRATCH_BYTES, stream);
}
