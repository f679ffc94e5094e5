// Batched products for int8 block-32 weights on the matrix cores: the
// ragged-batch decode path, where every sequence of the batch contributes one
// activation row and the batch is >= 16 rows, so Y = X . W^T is a dense
// contraction worth the MFMA units (below 16 rows the entry points run the
// matvec per row).
//
// Reference counterpart: gemm_f16 / gemm_gate_up_silu (KL/kernels.metal:376-510,
// host KL/main.swift:397-410), which the reference uses for prefill only, with
// fp16 weights. Arithmetic here: y[b][r] = sum over blocks of
// s[r][blk] * (sum over the block's 32 k of q[r][k] * x[b][k]) with x fp16, q
// int8 (exact in fp16), products exact in fp32 and fp32 accumulation.
//
// Work layout (gfx950, v_mfma_f32_32x32x16_f16):
//  * a workgroup of 4 waves owns 128 weight rows (32 per wave; for the
//    gate/up pair 64 rows of each matrix) x 64 activation rows (128 for large
//    fp16 prefill products, see pick_bt) x one split of K, walked in chunks
//    of 128 k (4 quantisation blocks);
//  * the weights are the B operand, so each lane's 16 results share one
//    weight row and one scale, and a lane's 16-byte load (row r, bytes
//    16h..16h+15 of a 32-byte block, h = lane / 32) feeds both MFMAs of the
//    block: bytes 0-7 pair with activation k 16h..16h+7 and bytes 8-15 with
//    16h+8..16h+15, so each MFMA's 16 k stay inside one block and
//    acc += s * (q . x) stays exact;
//  * weights go straight from HBM into registers two chunks ahead of the
//    math; activations are loaded into registers two chunks ahead and written
//    to a double-buffered LDS chunk (one barrier per chunk); the split's
//    scales sit in LDS from the start;
//  * the default kernel is fully unrolled over a compile-time number of chunks
//    (4, 8, 16 or 32), so every load is issued at a fixed point and the
//    compiler's waits are exact (a runtime loop carrying in-flight registers
//    gets a full drain at its head); a K whose chunk count no choice divides
//    runs the same layout as a runtime loop;
//  * K is split across workgroups; the fp32 partials are added in a fixed
//    order by a second kernel that also applies the epilogue, so results are
//    deterministic.
//
// Measured on MI355X at 64 rows (one Llama-3-8B layer, with the reduction):
// qkv 6144x4096 21.9 us, o 4096x4096 18.4 us, gate/up 2x14336x4096 62.2 us,
// down 4096x14336 34.8 us; an earlier layout (16x16 MFMAs, a 64 x 1024
// activation slice resident in LDS, one workgroup per CU) took 29.3 / 19.9 /
// 67.4 / 36.3 us.
#include "internal.hpp"

namespace {

constexpr int GM_WAVES = 4;
constexpr int GM_THREADS = GM_WAVES * 64;
constexpr int GM_ROWS = 32 * GM_WAVES;  // weight rows per workgroup (over both matrices)
constexpr int GM_BATCH = 64;            // activation rows per workgroup
constexpr int GM2_CK = 128;             // k per chunk (4 blocks)
constexpr int GM2_XP = GM2_CK + 8;      // LDS pitch in halfs of the runtime-loop kernel (+16 bytes)
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct GemmArgs {
    const int8_t* W[2];  // int8 [M][K], or fp16 [M][K] (MXD_W_F16) through the same pointer
    const uint16_t* S[2];
    const uint16_t* X;  // fp16 [n_rows][K]
    const float* Xf;    // or fp32 [n_rows][K], rounded to fp16 as it is staged (XF32 kernels)
    float* Y;           // fp32 [n_rows][M]
    uint16_t* Yh;       // or fp16 [n_rows][M] (nearest even), the store / activation epilogues only
    float* part;        // fp32 [splits][n_rows][NMAT][M] when splits > 1
    int n_rows, M, K, splits;
    int row_tiles, batch_tiles;  // weight-row tiles of GM_ROWS / NMAT, activation tiles of GM_BATCH
};

// XCD-aware tile order on a 1-D grid. Workgroup L runs on XCD L % 8 (the
// 8 XCDs take workgroups round-robin); the batch tiles of one (row tile,
// split) pair take consecutive slots of one XCD, so a weight tile streamed
// from HBM once is re-read from that XCD's L2 by the pair's other batch
// tiles, which run at the same time. The grid is rounded up to whole groups
// of 8 pairs; a workgroup past the last pair returns before any barrier.
__device__ __forceinline__ bool gemm_tile(const GemmArgs& a, int& split, int& rt, int& bz) {
    const int L = blockIdx.x, rest = L >> 3;
    bz = rest % a.batch_tiles;
    const int pair = (rest / a.batch_tiles) * 8 + (L & 7);
    if (pair >= a.row_tiles * a.splits) return false;
    rt = pair / a.splits;
    split = pair - rt * a.splits;
    return true;
}

template <int NMAT, int OP>
__device__ __forceinline__ float epilogue(float g, float u, float old) {
    if constexpr (NMAT == 2) {
        return (OP == MXD_ACT_SILU ? mxd::silu(g) : mxd::gelu_tanh(g)) * u;
    } else if constexpr (OP == MXD_EPI_ADD) {
        return old + g;
    } else {
        return g;
    }
}

// One 16-byte activation piece (8 k of one row) on its way to LDS: fp16 as
// loaded, or fp32 (two 16-byte loads) rounded to nearest-even fp16 when it is
// written (the rounding of mxd_f32_to_f16), so an fp32 producer needs no cast
// launch. e is the element offset of the piece in X.
template <bool XF32>
struct XPiece {
    u4_t v;
    __device__ __forceinline__ void load(const GemmArgs& a, size_t e) { v = *reinterpret_cast<const u4_t*>(a.X + e); }
    __device__ __forceinline__ u4_t h8() const { return v; }
};
template <>
struct XPiece<true> {
    f4_t lo, hi;
    __device__ __forceinline__ void load(const GemmArgs& a, size_t e) {
        lo = *reinterpret_cast<const f4_t*>(a.Xf + e);
        hi = *reinterpret_cast<const f4_t*>(a.Xf + e + 4);
    }
    static __device__ __forceinline__ uint32_t pack(float x, float y) {
        return (uint32_t)mxd::f2h_bits(x) | ((uint32_t)mxd::f2h_bits(y) << 16);
    }
    __device__ __forceinline__ u4_t h8() const {
        return u4_t{pack(lo.x, lo.y), pack(lo.z, lo.w), pack(hi.x, hi.y), pack(hi.z, hi.w)};
    }
};

__device__ __forceinline__ h8_t q8x8_to_h8(uint32_t lo, uint32_t hi) {
    h2_t a[4];
    mxd::i8x4_to_h2x2(lo, a[0], a[1]);
    mxd::i8x4_to_h2x2(hi, a[2], a[3]);
    return h8_t{a[0].x, a[0].y, a[1].x, a[1].y, a[2].x, a[2].y, a[3].x, a[3].y};
}

// Eight dequantised weights fp16(q * s): the int8 values are exact in fp16,
// and each product is rounded once (packed fp16 multiplies), so the matrix
// cores accumulate the scaled weights directly.
__device__ __forceinline__ h8_t q8x8_scaled(uint32_t lo, uint32_t hi, _Float16 s) {
    const h8_t q = q8x8_to_h8(lo, hi);
    const h8_t sv = {s, s, s, s, s, s, s, s};
    return q * sv;
}

// The runtime-loop form (any chunk count): activations in registers two
// chunks ahead, a register ring of two chunks of weights and scales.
template <int NMAT, int OP, bool XF32>
__global__ void __launch_bounds__(GM_THREADS) gemm_q8_loop_kernel(GemmArgs a) {
    constexpr int WAVES = GM_WAVES, NT = GM_THREADS;
    constexpr int WPM = WAVES / NMAT;  // waves per matrix
    constexpr int ROWS = 32 * WPM;     // weight rows of each matrix per workgroup
    constexpr int XPT = GM_BATCH * GM2_CK / 8 / NT;  // 16-byte activation pieces per thread per chunk
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][GM_BATCH][GM2_XP];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int mc = lane & 31, h = lane >> 5;
    const int m = wave / WPM;  // which matrix this wave reads
    int split, rt, bz;
    if (!gemm_tile(a, split, rt, bz)) return;
    const int row0 = rt * ROWS + 32 * (wave % WPM);
    const int b0 = bz * GM_BATCH;
    const int M = a.M, K = a.K;
    const int nck = K / GM2_CK;
    const int c0 = split * nck / a.splits, c1 = (split + 1) * nck / a.splits;  // this split's chunks

    // Weight row mc of the wave's 32 (clamped past M: computed, never stored).
    const int wrow = min(row0 + mc, M - 1);
    const int8_t* wp = a.W[m] + (size_t)wrow * K + (size_t)c0 * GM2_CK + 16 * h;
    const uint16_t* sp = a.S[m] + (size_t)wrow * (K / 32) + (size_t)c0 * 4;
    // Ring of two chunks: slot (par, j) holds block j of chunk c0 + 2i + par.
    u4_t wr[2][4];
    u2_t sr[2];
#pragma unroll
    for (int par = 0; par < 2; ++par) {
        if (c0 + par < c1) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wr[par][j] = *reinterpret_cast<const u4_t*>(wp + (size_t)par * GM2_CK + 32 * j);
            sr[par] = *reinterpret_cast<const u2_t*>(sp + 4 * par);
        }
    }

    // Activation chunk c: 64 rows x 128 halfs as 1024 pieces of 16 bytes;
    // thread t takes pieces t + NT u (row p / 16, piece p % 16). Rows past
    // n_rows are stored as zeros (loaded from a clamped, valid row).
    const size_t xoff = (size_t)c0 * GM2_CK;
    auto load_x = [&](XPiece<XF32> (&v)[XPT], int ci) {
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int p = threadIdx.x + NT * u, r = p >> 4, q = p & 15;
            v[u].load(a, xoff + (size_t)min(b0 + r, a.n_rows - 1) * K + (size_t)ci * GM2_CK + 8 * q);
        }
    };
    auto store_x = [&](const XPiece<XF32> (&v)[XPT], int buf) {
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int p = threadIdx.x + NT * u, r = p >> 4, q = p & 15;
            const u4_t z = {0u, 0u, 0u, 0u};
            *reinterpret_cast<u4_t*>(&xs[buf][r][8 * q]) = b0 + r < a.n_rows ? v[u].h8() : z;
        }
    };
    // Register ring of two chunks: set p holds chunk ci (ci & 1 == p) from its
    // load, issued two chunks ahead, until it is stored to LDS buffer p at the
    // end of chunk ci - 1.
    XPiece<XF32> xv[2][XPT];
    load_x(xv[0], 0);
    if (c0 + 1 < c1) load_x(xv[1], 1);
    store_x(xv[0], 0);
    __syncthreads();

    f32x16_t acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

    // One chunk (ci = chunk index within the split, par = ci & 1, also the LDS
    // buffer holding it).
    auto chunk = [&](const int ci, const int par) {
        const bool more = c0 + ci + 1 < c1;
        if (c0 + ci + 2 < c1) load_x(xv[par], ci + 2);
        _Float16 sc[4];
        {
            const u2_t sv = sr[par];
            sc[0] = mxd::as_h2(sv.x).x;
            sc[1] = mxd::as_h2(sv.x).y;
            sc[2] = mxd::as_h2(sv.y).x;
            sc[3] = mxd::as_h2(sv.y).y;
        }
        const bool refill = c0 + ci + 2 < c1;
        if (refill) sr[par] = *reinterpret_cast<const u2_t*>(sp + 4 * (ci + 2));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u4_t w = wr[par][j];
            if (refill)
                wr[par][j] = *reinterpret_cast<const u4_t*>(
                    wp + (size_t)(ci + 2) * GM2_CK + 32 * j);
            const h8_t w0 = q8x8_scaled(w.x, w.y, sc[j]), w1 = q8x8_scaled(w.z, w.w, sc[j]);
            const int kx = 32 * j + 16 * h;
            const h8_t x00 = *reinterpret_cast<const h8_t*>(&xs[par][mc][kx]);
            const h8_t x01 = *reinterpret_cast<const h8_t*>(&xs[par][mc][kx + 8]);
            const h8_t x10 = *reinterpret_cast<const h8_t*>(&xs[par][32 + mc][kx]);
            const h8_t x11 = *reinterpret_cast<const h8_t*>(&xs[par][32 + mc][kx + 8]);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x00, w0, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x10, w0, acc[1], 0, 0, 0);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x01, w1, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x11, w1, acc[1], 0, 0, 0);
        }
        if (more) store_x(xv[par ^ 1], par ^ 1);
        __syncthreads();
    };
    const int nc = c1 - c0;
    for (int ci = 0; ci < nc; ci += 2) {
        chunk(ci, 0);
        if (ci + 1 < nc) chunk(ci + 1, 1);
    }

    // Lane (mc, h), register r of tile t: activation row b0 + 32 t + 8 (r / 4)
    // + 4 h + r % 4, weight row row0 + mc.
    const int wr_out = row0 + mc;
    auto brow = [&](int t, int r) { return b0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3); };
    if (a.splits > 1) {
        if (wr_out < M) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int b = brow(t, r);
                    if (b < a.n_rows) a.part[(((size_t)split * a.n_rows + b) * NMAT + m) * M + wr_out] = acc[t][r];
                }
        }
        return;
    }
    if constexpr (NMAT == 2) {
        // The up waves hand their sums to the gate waves of the same rows
        // through LDS (the activation buffers are free after the last barrier).
        float* xf = reinterpret_cast<float*>(&xs[0][0][0]);
        if (m == 1) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) xf[(((wave - WPM) * 2 + t) * 16 + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (m == 1 || wr_out >= M) return;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int b = brow(t, r);
                const float u = xf[((wave * 2 + t) * 16 + r) * 64 + lane];
                if (b < a.n_rows) a.Y[(size_t)b * M + wr_out] = epilogue<NMAT, OP>(acc[t][r], u, 0.0f);
            }
    } else {
        if (wr_out >= M) return;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int b = brow(t, r);
                if (b < a.n_rows) {
                    float* y = a.Y + (size_t)b * M + wr_out;
                    *y = epilogue<NMAT, OP>(acc[t][r], 0.0f, OP == MXD_EPI_ADD ? *y : 0.0f);
                }
            }
    }
}

// Compile-time loop helpers for the fully unrolled chunk loop below.
template <int V>
struct ic {
    static constexpr int value = V;
};
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(ic<I>{});
        static_for<I + 1, N>(f);
    }
}

// The default kernel: NCH chunks per workgroup, fully unrolled. WF selects
// the weights: int8 block-32 (a lane's 16-byte load is half a block, dequantised
// and scaled per block) or fp16 (a lane's 16 k of a block are 32 contiguous
// bytes, two 16-byte loads that are the MFMA operands as they stand; products
// accumulate in the MFMA accumulators). The k order, the activation side and
// the epilogues are the same for both.
// At 128 activation rows the kernel asks for two waves per SIMD (256 VGPRs;
// the compiler spills 2 dwords per lane at 8-16 chunks): left to itself it
// took 257-280 registers and one wave per SIMD, and the two-wave form ran
// gate/up 2 x 16384 x 2048 at 512 / 1024 rows in 117.6 / 197 us against 142 /
// 260 (measured on MI355X).
template <int WF, int NMAT, int OP, int NCH, bool XF32, int BT = GM_BATCH>
__global__ void __launch_bounds__(GM_THREADS, BT == 128 ? 2 : 1) gemm_mfma_kernel(GemmArgs a) {
    constexpr int WAVES = GM_WAVES, NT = GM_THREADS;
    constexpr int WPM = WAVES / NMAT;
    constexpr int ROWS = 32 * WPM;
    constexpr int NB = BT / 32;  // 32-row activation tiles: MFMAs per weight operand
    constexpr int XPT = BT * GM2_CK / 8 / NT;
    // Two activation buffers (chunk ci in xs[ci & 1]), rows swizzled: piece p
    // of row b sits at slot p ^ (b & 15).
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][BT][GM2_CK];
    // the split's scales of each wave's 32 rows: [wave][row][NCH * 4 (+8 pad,
    // keeping every row 16-byte aligned for the 16-byte stores below)]
    constexpr bool Q8 = WF == MXD_W_Q8B32;
    constexpr int SP = Q8 ? NCH * 4 + 8 : 8;
    __shared__ __attribute__((aligned(16))) uint16_t ss[WAVES][32][SP];
    constexpr int ESZ = Q8 ? 1 : 2;  // bytes per weight

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int mc = lane & 31, h = lane >> 5;
    const int m = wave / WPM;
    int split, rt, bz;
    if (!gemm_tile(a, split, rt, bz)) return;
    const int row0 = rt * ROWS + 32 * (wave % WPM);
    const int b0 = bz * BT;
    const int M = a.M, K = a.K;
    const int c0 = split * NCH;  // a.splits * NCH == K / GM2_CK

    const int wrow = min(row0 + mc, M - 1);
    const unsigned char* wp =
        reinterpret_cast<const unsigned char*>(a.W[m]) + ((size_t)wrow * K + (size_t)c0 * GM2_CK + 16 * h) * ESZ;
    const size_t xoff = (size_t)c0 * GM2_CK;

    // Activations of chunk ci: thread t loads pieces t + NT u (row p / 16,
    // piece p % 16) into register set ci & 1, two chunks ahead; the set is
    // written to LDS buffer ci & 1 at the end of chunk ci - 1.
    XPiece<XF32> xv[2][XPT];
    auto load_x = [&](auto cic) {
        constexpr int ci = decltype(cic)::value;
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int p = threadIdx.x + NT * u, r = p >> 4, q = p & 15;
            xv[ci & 1][u].load(a, xoff + (size_t)min(b0 + r, a.n_rows - 1) * K + (size_t)ci * GM2_CK + 8 * q);
        }
    };
    auto store_x = [&](auto cic) {
        constexpr int ci = decltype(cic)::value;
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int p = threadIdx.x + NT * u, r = p >> 4, q = p & 15;
            *reinterpret_cast<u4_t*>(&xs[ci & 1][r][8 * (q ^ (r & 15))]) = xv[ci & 1][u].h8();
        }
    };
    // Block j of chunk ci: ESZ 16-byte pieces per lane. Ordinary (temporal)
    // loads: a wave reads each 128-byte line of a weight row as four 32-byte
    // pieces, one per block, so the line must stay in L2 until the fourth;
    // with nontemporal loads L2 refetched lines (FETCH_SIZE 1.27x the weight
    // bytes) and the products ran ~20% slower (gate/up 55.6 -> 44.9 us at 64
    // rows).
    u4_t wr[2][4 * ESZ];
    auto load_w = [&](int ci, int j) {
#pragma unroll
        for (int e = 0; e < ESZ; ++e)
            wr[ci & 1][ESZ * j + e] =
                *reinterpret_cast<const u4_t*>(wp + ((size_t)ci * GM2_CK + 32 * j) * ESZ + 16 * e);
    };
    // int8: scales first; lane l fetches row l / 2's half (l & 1) of the
    // split's NCH * 4 scales (NCH * 4 bytes) in 16-byte pieces.
    constexpr int SPL = Q8 ? NCH * 4 / 2 / 8 : 1;  // 16-byte pieces per lane
    u4_t sv[SPL];
    if constexpr (Q8) {
        const uint16_t* srow = a.S[m] + (size_t)min(row0 + (lane >> 1), M - 1) * (K / 32) + (size_t)c0 * 4 +
                               (lane & 1) * (NCH * 2);
#pragma unroll
        for (int u = 0; u < SPL; ++u) sv[u] = *reinterpret_cast<const u4_t*>(srow + 8 * u);
    }
    // Every load lands in registers, so the compiler's own waits are exact.
    load_x(ic<0>{});
#pragma unroll
    for (int j = 0; j < 4; ++j) load_w(0, j);
    if constexpr (NCH > 1) {
        load_x(ic<1>{});
#pragma unroll
        for (int j = 0; j < 4; ++j) load_w(1, j);
    }
    if constexpr (Q8) {
#pragma unroll
        for (int u = 0; u < SPL; ++u)
            *reinterpret_cast<u4_t*>(&ss[wave][lane >> 1][(lane & 1) * (NCH * 2) + 8 * u]) = sv[u];
    }
    store_x(ic<0>{});
    __syncthreads();
    f32x16_t acc[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

    static_for<0, NCH>([&](auto cic) {
        constexpr int ci = decltype(cic)::value;
        constexpr int par = ci & 1;
        const _Float16(*xcur)[GM2_CK] = xs[par];
        _Float16 sc[4];
        if constexpr (Q8) {
            const u2_t sv2 = *reinterpret_cast<const u2_t*>(&ss[wave][mc][4 * ci]);
            sc[0] = mxd::as_h2(sv2.x).x;
            sc[1] = mxd::as_h2(sv2.x).y;
            sc[2] = mxd::as_h2(sv2.y).x;
            sc[3] = mxd::as_h2(sv2.y).y;
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (ci + 2 < NCH) load_x(ic<ci + 2>{});
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h8_t w0, w1;
            if constexpr (Q8) {
                const u4_t w = wr[par][j];
                w0 = q8x8_scaled(w.x, w.y, sc[j]);
                w1 = q8x8_scaled(w.z, w.w, sc[j]);
            } else {
                __builtin_memcpy(&w0, &wr[par][2 * j], 16);
                __builtin_memcpy(&w1, &wr[par][2 * j + 1], 16);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (ci + 2 < NCH) load_w(ci + 2, j);
            __builtin_amdgcn_sched_barrier(0);
            const int p0 = 4 * j + 2 * h, sw = mc & 15;
            // (32t + mc) & 15 == mc & 15: one swizzle for every activation tile
            h8_t x0[NB], x1[NB];
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                x0[t] = *reinterpret_cast<const h8_t*>(&xcur[32 * t + mc][8 * (p0 ^ sw)]);
                x1[t] = *reinterpret_cast<const h8_t*>(&xcur[32 * t + mc][8 * ((p0 + 1) ^ sw)]);
            }
#pragma unroll
            for (int t = 0; t < NB; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0[t], w0, acc[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NB; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1[t], w1, acc[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NB; ++t) asm volatile("" : "+v"(acc[t]));
        }
        if constexpr (ci + 1 < NCH) {
            store_x(ic<ci + 1>{});
            __syncthreads();
        }
    });

    const int wr_out = row0 + mc;
    auto brow = [&](int t, int r) { return b0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3); };
    if (a.splits > 1) {
        if (wr_out < M) {
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int b = brow(t, r);
                    if (b < a.n_rows) a.part[(((size_t)split * a.n_rows + b) * NMAT + m) * M + wr_out] = acc[t][r];
                }
        }
        return;
    }
    if constexpr (NMAT == 2) {
        // WPM * NB * 1024 floats (16 KiB at 64 rows, 32 KiB at 128), inside xs
        static_assert(WPM * NB * 1024 * sizeof(float) <= sizeof(xs), "epilogue scratch exceeds the LDS buffer");
        float* xf = reinterpret_cast<float*>(&xs[0][0][0]);
        __syncthreads();  // every wave is past its last LDS read
        if (m == 1) {
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) xf[(((wave - WPM) * NB + t) * 16 + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (m == 1 || wr_out >= M) return;
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int b = brow(t, r);
                const float u = xf[((wave * NB + t) * 16 + r) * 64 + lane];
                if (b < a.n_rows) {
                    const float y = epilogue<NMAT, OP>(acc[t][r], u, 0.0f);
                    if (a.Yh)
                        a.Yh[(size_t)b * M + wr_out] = mxd::f2h_bits(y);
                    else
                        a.Y[(size_t)b * M + wr_out] = y;
                }
            }
    } else {
        if (wr_out >= M) return;
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int b = brow(t, r);
                if (b < a.n_rows) {
                    float* y = a.Y + (size_t)b * M + wr_out;
                    *y = epilogue<NMAT, OP>(acc[t][r], 0.0f, OP == MXD_EPI_ADD ? *y : 0.0f);
                }
            }
    }
}

// Y[b][r] = epilogue(sum over splits, in split order) of the partials.
template <int NMAT, int OP>
__global__ void __launch_bounds__(256) gemm_reduce_kernel(GemmArgs a) {
    const size_t n = (size_t)a.n_rows * a.M;
    const size_t stride = (size_t)a.n_rows * NMAT * a.M;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256) {
        const size_t b = e / a.M, r = e - b * a.M;
        const float* p = a.part + b * NMAT * a.M + r;
        float s0 = 0.0f, s1 = 0.0f;
        for (int sp = 0; sp < a.splits; ++sp) {
            s0 += p[sp * stride];
            if (NMAT == 2) s1 += p[sp * stride + a.M];
        }
        if (NMAT == 2 && a.Yh)
            a.Yh[e] = mxd::f2h_bits(epilogue<NMAT, OP>(s0, s1, 0.0f));
        else
            a.Y[e] = epilogue<NMAT, OP>(s0, s1, OP == MXD_EPI_ADD && NMAT == 1 ? a.Y[e] : 0.0f);
    }
}

// Both weight formats need whole 128-k chunks: int8 runs any chunk count
// (the runtime loop takes the ones the unrolled kernel does not), fp16 runs
// the unrolled kernel only, with 1 or 2 chunks per workgroup where 4 does not
// divide the count (K = 128, 256, 384, ...: Gemma-4's per-layer-input
// projection back to the model width has K = 256).
bool use_mfma(int wf, int n_rows, int K) {
    (void)wf;
    return n_rows >= mxd::tunable("GM_MIN_ROWS", 16) && K % GM2_CK == 0;
}

// Chunks per workgroup of the unrolled kernel: the largest of 32, 16, 8, 4
// that divides K's chunk count and still gives at least 128 workgroups (half
// the CUs: fewer, longer splits write fewer partials; the 4096 x 4096 product
// at 64 rows ran 15.7 us as 4 splits of 8 chunks against 16.6 us as 8 of 4);
// the GM_NCH tunable (4, 8, 16, 32) forces one, GM_NCH = 1 the runtime
// loop; 0 (the runtime loop) when none divides. Fewer, longer splits also save
// the partials and their reduction (gate/up at 64 rows: 62.2 us with one split
// of 32 chunks against 65.1 us with two of 16).
int pick_nch(int wf, int n_rows, int M, int K, int nmat, int bt) {
    const int nck = K / GM2_CK;
    const int tiles = ((M + GM_ROWS / nmat - 1) / (GM_ROWS / nmat)) * ((n_rows + bt - 1) / bt);
    const int forced = mxd::tunable("GM_NCH", 0);
    const bool loop_ok = wf == MXD_W_Q8B32;  // the runtime-loop kernel is int8 only
    if (forced == 1 && loop_ok) return 0;
    if ((forced == 4 || forced == 8 || forced == 16 || forced == 32) && (nck % forced == 0 || loop_ok))
        return nck % forced == 0 ? forced : 0;
    // fp16 also has 12 and 6 chunks per workgroup, for K = 1536 (Gemma-4-E2B)
    // and its multiples: one or two splits instead of three, whose reduction
    // read three partials per output (E2B gate/up at 512 rows: 20.9 us).
    const bool f16 = wf == MXD_W_F16;
    int best = 0;
    for (int nch : {32, 16, 12, 8, 6, 4}) {
        if (nck % nch || (!f16 && nch % 4 == 2) || (!f16 && nch == 12)) continue;
        if (!best) best = nch;
        if (tiles * (nck / nch) >= 128) return nch;
        best = nch;
    }
    if (!best && f16) best = nck % 2 == 0 ? 2 : 1;  // fp16 has no runtime loop
    return best;
}

// K splits: nck / NCH for the unrolled kernel; for the runtime loop about two
// workgroups per CU, at most one split per chunk. GM_SPLITS overrides the
// latter.
int pick_splits(int wf, int n_rows, int M, int K, int nmat, int bt = GM_BATCH) {
    const int nch = pick_nch(wf, n_rows, M, K, nmat, bt);
    if (nch) return (K / GM2_CK) / nch;
    const int tiles = ((M + GM_ROWS / nmat - 1) / (GM_ROWS / nmat)) * ((n_rows + bt - 1) / bt);
    const int s = mxd::tunable("GM_SPLITS", (512 + tiles - 1) / tiles);
    return max(1, min(s, K / GM2_CK));
}

// Activation rows per workgroup: 128 for fp16 weights against fp16
// activations from 256 rows on while that leaves 128 or more tiles (half the
// CUs), and from 512 rows on while it leaves GM_BT_TILES (16) or more, so each
// weight operand feeds four MFMAs; else 64 (int8 weights, fp32 activations:
// their staging registers would not fit at 128). Measured on MI355X: gate/up
// 2 x 16384 x 2048 at 256 / 512 / 1024 rows 68.9 / 129.7 / 254 us against
// 79.7 / 138.4 / 269 at 64; down 2048 x 16384 at 512 rows 59.6 against 77.1.
// Alone, q|k|v 2560 x 2048 and o 2048 x 2048 at 512 rows ran slower at 128
// (25.2 / 22.5 against 20.8 / 19.2 us), but the Gemma-2B pp512 prefill ran
// 102.6-103.1k tok/s with every product at 128 rows against 93.6-94.0k with
// only gate/up at 128 (E2B pp512 57.0k against 54.3k); at 256 rows every
// product at 128 ran pp256 at 67.7k against 74.0k. GM_BT = 64 keeps 64.
int pick_bt(int wf, bool xf32, int n_rows, int M, int nmat) {
    if (wf != MXD_W_F16 || xf32 || n_rows < 256 || mxd::tunable("GM_BT", 128) == 64) return GM_BATCH;
    const int tiles = ((M + GM_ROWS / nmat - 1) / (GM_ROWS / nmat)) * ((n_rows + 127) / 128);
    if (tiles >= 128) return 128;
    return n_rows >= 512 && tiles >= mxd::tunable("GM_BT_TILES", 16) ? 128 : GM_BATCH;
}

// The workspace of either activation dtype (the size queries do not know it).
size_t ws_bytes_for(int wf, int n_rows, int M, int K, int nmat) {
    if (n_rows <= 0 || M <= 0 || K <= 0 || !use_mfma(wf, n_rows, K)) return 0;
    size_t need = 0;
    for (const int bt : {pick_bt(wf, true, n_rows, M, nmat), pick_bt(wf, false, n_rows, M, nmat)}) {
        const int s = pick_splits(wf, n_rows, M, K, nmat, bt);
        if (s > 1) need = max(need, (size_t)s * n_rows * nmat * M * sizeof(float));
    }
    return need;
}

// With defer set, the K-split partials are the result: they go to ws as
// [splits][n_rows][NMAT][M] (a single split stores its product there as
// split 0) and the sum is left to the consumer.
template <int WF, int NMAT, int OP, bool XF32 = false>
int launch_gemm(GemmArgs a, void* ws, size_t ws_bytes, hipStream_t s, const char* fn, bool defer = false) {
    const int bt = pick_bt(WF, XF32, a.n_rows, a.M, NMAT);
    a.splits = pick_splits(WF, a.n_rows, a.M, a.K, NMAT, bt);
    const size_t need =
        a.splits > 1 || defer ? (size_t)a.splits * a.n_rows * NMAT * a.M * sizeof(float) : 0;
    MXD_REQUIRE(need == 0 || (ws && ws_bytes >= need), MXD_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)",
                fn, need, ws_bytes);
    a.part = static_cast<float*>(ws);
    if (defer && a.splits == 1) a.Y = a.part;
    a.row_tiles = (a.M + GM_ROWS / NMAT - 1) / (GM_ROWS / NMAT);
    a.batch_tiles = (a.n_rows + bt - 1) / bt;
    const int pairs = a.row_tiles * a.splits;
    const dim3 grid((unsigned)((pairs + 7) / 8 * 8 * a.batch_tiles));  // see gemm_tile
    const int nch = pick_nch(WF, a.n_rows, a.M, a.K, NMAT, bt);
    if constexpr (WF == MXD_W_F16 && !XF32) {
        if (bt == 128) {
            switch (nch) {
                case 1: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 1, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 2: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 2, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 4: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 4, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 8: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 8, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 16: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 16, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 6: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 6, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 12: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 12, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                case 32: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 32, XF32, 128>), grid, dim3(GM_THREADS), 0, s, a); break;
                default: return mxd::fail(MXD_ERR_UNSUPPORTED, "%s: K=%d has no chunk count for fp16 weights", fn, a.K);
            }
            if (a.splits > 1 && !defer) {
                const size_t n = (size_t)a.n_rows * a.M;
                const size_t nb = (n + 255) / 256;
                const unsigned blocks = (unsigned)(nb < 4096 ? nb : 4096);
                hipLaunchKernelGGL((gemm_reduce_kernel<NMAT, OP>), dim3(blocks), dim3(256), 0, s, a);
            }
            return mxd::check_launch(fn);
        }
    }
    switch (nch) {
        case 4: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 4, XF32>), grid, dim3(GM_THREADS), 0, s, a); break;
        case 8: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 8, XF32>), grid, dim3(GM_THREADS), 0, s, a); break;
        case 16: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 16, XF32>), grid, dim3(GM_THREADS), 0, s, a); break;
        case 32: hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 32, XF32>), grid, dim3(GM_THREADS), 0, s, a); break;
        case 12:
        case 6:
        case 2:
        case 1:
            if constexpr (WF == MXD_W_F16) {
                if (nch == 12)
                    hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 12, XF32>), grid, dim3(GM_THREADS), 0, s, a);
                else if (nch == 6)
                    hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 6, XF32>), grid, dim3(GM_THREADS), 0, s, a);
                else if (nch == 2)
                    hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 2, XF32>), grid, dim3(GM_THREADS), 0, s, a);
                else
                    hipLaunchKernelGGL((gemm_mfma_kernel<WF, NMAT, OP, 1, XF32>), grid, dim3(GM_THREADS), 0, s, a);
                break;
            }
            [[fallthrough]];
        default:
            if constexpr (WF == MXD_W_Q8B32) {
                hipLaunchKernelGGL((gemm_q8_loop_kernel<NMAT, OP, XF32>), grid, dim3(GM_THREADS), 0, s, a);
            } else {
                return mxd::fail(MXD_ERR_UNSUPPORTED, "%s: K=%d has no chunk count for fp16 weights", fn, a.K);
            }
            break;
    }
    if (a.splits > 1 && !defer) {
        const size_t n = (size_t)a.n_rows * a.M;
        const size_t nb = (n + 255) / 256;
        const unsigned blocks = (unsigned)(nb < 4096 ? nb : 4096);
        hipLaunchKernelGGL((gemm_reduce_kernel<NMAT, OP>), dim3(blocks), dim3(256), 0, s, a);
    }
    return mxd::check_launch(fn);
}

int check_common(const void* W, const void* S, const void* X, const void* Y, int n_rows, int M, int K, const char* fn) {
    MXD_REQUIRE(W && S && X && Y, MXD_ERR_INVALID_ARG, "%s: null pointer", fn);
    MXD_REQUIRE(n_rows > 0 && M > 0 && K > 0, MXD_ERR_INVALID_ARG, "%s: n_rows=%d M=%d K=%d must be positive", fn,
                n_rows, M, K);
    MXD_REQUIRE(K % 32 == 0, MXD_ERR_INVALID_ARG, "%s: K=%d must be a multiple of 32 (quantisation blocks)", fn, K);
    const uintptr_t al = reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(S) |
                         reinterpret_cast<uintptr_t>(X);
    MXD_REQUIRE((al & 15) == 0, MXD_ERR_UNSUPPORTED, "%s: W, scales and X must be 16-byte aligned", fn);
    return MXD_OK;
}

}  // namespace

extern "C" size_t mxd_gemm_q8b32_workspace_size(int n_rows, int M, int K) {
    return ws_bytes_for(MXD_W_Q8B32, n_rows, M, K, 1);
}

extern "C" size_t mxd_gemm_gate_up_q8b32_workspace_size(int n_rows, int F, int K) {
    return ws_bytes_for(MXD_W_Q8B32, n_rows, F, K, 2);
}

extern "C" size_t mxd_gemm_f16_workspace_size(int n_rows, int M, int K) {
    return ws_bytes_for(MXD_W_F16, n_rows, M, K, 1);
}

extern "C" size_t mxd_gemm_gate_up_f16_workspace_size(int n_rows, int F, int K) {
    return ws_bytes_for(MXD_W_F16, n_rows, F, K, 2);
}

extern "C" int mxd_gemm_q8b32(const int8_t* Wq, const uint16_t* scales, const void* X, int x_dtype, float* Y,
                              int n_rows, int M, int K, int epilogue, void* workspace, size_t ws_bytes,
                              mxd_stream_t stream) {
    if (int rc = check_common(Wq, scales, X, Y, n_rows, M, K, "mxd_gemm_q8b32")) return rc;
    MXD_REQUIRE(epilogue == MXD_EPI_STORE || epilogue == MXD_EPI_ADD, MXD_ERR_INVALID_ARG,
                "mxd_gemm_q8b32: epilogue %d (store or add)", epilogue);
    MXD_REQUIRE(x_dtype == MXD_F16 || x_dtype == MXD_F32, MXD_ERR_INVALID_ARG, "mxd_gemm_q8b32: x_dtype %d",
                x_dtype);
    const size_t xesz = x_dtype == MXD_F32 ? 4 : 2;
    if (!use_mfma(MXD_W_Q8B32, n_rows, K)) {  // few rows: one matvec per row (fp32 X rounded the same way)
        for (int b = 0; b < n_rows; ++b) {
            const void* xb = static_cast<const char*>(X) + (size_t)b * K * xesz;
            const int rc = x_dtype == MXD_F32
                               ? mxd::matvec_xr16(MXD_W_Q8B32, Wq, scales, static_cast<const float*>(xb),
                                                  Y + (size_t)b * M, M, K, epilogue, mxd::as_stream(stream))
                               : mxd_matvec_q8b32(Wq, scales, xb, MXD_F16, Y + (size_t)b * M, M, K, epilogue, nullptr,
                                                  stream);
            if (rc) return rc;
        }
        return MXD_OK;
    }
    GemmArgs a{};
    a.W[0] = a.W[1] = Wq;
    a.S[0] = a.S[1] = scales;
    a.X = static_cast<const uint16_t*>(X);
    a.Xf = static_cast<const float*>(X);
    a.Y = Y;
    a.n_rows = n_rows;
    a.M = M;
    a.K = K;
    hipStream_t s = mxd::as_stream(stream);
    if (x_dtype == MXD_F32) {
        if (epilogue == MXD_EPI_ADD)
            return launch_gemm<MXD_W_Q8B32, 1, MXD_EPI_ADD, true>(a, workspace, ws_bytes, s, "mxd_gemm_q8b32");
        return launch_gemm<MXD_W_Q8B32, 1, MXD_EPI_STORE, true>(a, workspace, ws_bytes, s, "mxd_gemm_q8b32");
    }
    if (epilogue == MXD_EPI_ADD)
        return launch_gemm<MXD_W_Q8B32, 1, MXD_EPI_ADD>(a, workspace, ws_bytes, s, "mxd_gemm_q8b32");
    return launch_gemm<MXD_W_Q8B32, 1, MXD_EPI_STORE>(a, workspace, ws_bytes, s, "mxd_gemm_q8b32");
}

extern "C" size_t mxd_gemm_q8b32_partials_size(int n_rows, int M, int K) {
    if (n_rows <= 0 || M <= 0 || K <= 0 || K % 32 != 0 || !use_mfma(MXD_W_Q8B32, n_rows, K)) return 0;
    return (size_t)pick_splits(MXD_W_Q8B32, n_rows, M, K, 1) * n_rows * M * sizeof(float);
}

extern "C" int mxd_gemm_q8b32_partials(const int8_t* Wq, const uint16_t* scales, const void* X, int x_dtype,
                                       float* part, size_t part_bytes, int n_rows, int M, int K, int* n_splits,
                                       mxd_stream_t stream) {
    if (int rc = check_common(Wq, scales, X, part, n_rows, M, K, "mxd_gemm_q8b32_partials")) return rc;
    MXD_REQUIRE(n_splits, MXD_ERR_INVALID_ARG, "mxd_gemm_q8b32_partials: n_splits is null");
    MXD_REQUIRE(x_dtype == MXD_F16 || x_dtype == MXD_F32, MXD_ERR_INVALID_ARG, "mxd_gemm_q8b32_partials: x_dtype %d",
                x_dtype);
    MXD_REQUIRE(use_mfma(MXD_W_Q8B32, n_rows, K), MXD_ERR_UNSUPPORTED,
                "mxd_gemm_q8b32_partials: n_rows=%d K=%d is not a matrix-core product (16+ rows, K %% 128 == 0)",
                n_rows, K);
    GemmArgs a{};
    a.W[0] = a.W[1] = Wq;
    a.S[0] = a.S[1] = scales;
    a.X = static_cast<const uint16_t*>(X);
    a.Xf = static_cast<const float*>(X);
    a.Y = part;
    a.n_rows = n_rows;
    a.M = M;
    a.K = K;
    *n_splits = pick_splits(MXD_W_Q8B32, n_rows, M, K, 1);
    hipStream_t s = mxd::as_stream(stream);
    if (x_dtype == MXD_F32)
        return launch_gemm<MXD_W_Q8B32, 1, MXD_EPI_STORE, true>(a, part, part_bytes, s, "mxd_gemm_q8b32_partials",
                                                                 true);
    return launch_gemm<MXD_W_Q8B32, 1, MXD_EPI_STORE>(a, part, part_bytes, s, "mxd_gemm_q8b32_partials", true);
}

extern "C" int mxd_gemm_gate_up_q8b32(const int8_t* Wg, const uint16_t* sg, const int8_t* Wu, const uint16_t* su,
                                      const uint16_t* X, float* H, int n_rows, int F, int K, int act, void* workspace,
                                      size_t ws_bytes, mxd_stream_t stream) {
    if (int rc = check_common(Wg, sg, X, H, n_rows, F, K, "mxd_gemm_gate_up_q8b32")) return rc;
    if (int rc = check_common(Wu, su, X, H, n_rows, F, K, "mxd_gemm_gate_up_q8b32")) return rc;
    MXD_REQUIRE(act == MXD_ACT_GELU_TANH || act == MXD_ACT_SILU, MXD_ERR_INVALID_ARG,
                "mxd_gemm_gate_up_q8b32: unknown activation %d", act);
    if (!use_mfma(MXD_W_Q8B32, n_rows, K)) {
        for (int b = 0; b < n_rows; ++b) {
            if (int rc = mxd_matvec_gate_up(MXD_W_Q8B32, Wg, sg, Wu, su, X + (size_t)b * K, MXD_F16, H + (size_t)b * F,
                                            F, K, act, stream))
                return rc;
        }
        return MXD_OK;
    }
    GemmArgs a{};
    a.W[0] = Wg;
    a.W[1] = Wu;
    a.S[0] = sg;
    a.S[1] = su;
    a.X = X;
    a.Y = H;
    a.n_rows = n_rows;
    a.M = F;
    a.K = K;
    hipStream_t s = mxd::as_stream(stream);
    if (act == MXD_ACT_SILU)
        return launch_gemm<MXD_W_Q8B32, 2, MXD_ACT_SILU>(a, workspace, ws_bytes, s, "mxd_gemm_gate_up_q8b32");
    return launch_gemm<MXD_W_Q8B32, 2, MXD_ACT_GELU_TANH>(a, workspace, ws_bytes, s, "mxd_gemm_gate_up_q8b32");
}

namespace {

int check_f16(const void* W, const void* X, const void* Y, int n_rows, int M, int K, const char* fn) {
    MXD_REQUIRE(W && X && Y, MXD_ERR_INVALID_ARG, "%s: null pointer", fn);
    MXD_REQUIRE(n_rows > 0 && M > 0 && K > 0, MXD_ERR_INVALID_ARG, "%s: n_rows=%d M=%d K=%d must be positive", fn,
                n_rows, M, K);
    MXD_REQUIRE(K % 8 == 0, MXD_ERR_INVALID_ARG, "%s: K=%d must be a multiple of 8", fn, K);
    const uintptr_t al = reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(X);
    MXD_REQUIRE((al & 15) == 0, MXD_ERR_UNSUPPORTED, "%s: W and X must be 16-byte aligned", fn);
    return MXD_OK;
}

}  // namespace

extern "C" int mxd_gemm_f16(const uint16_t* W, const void* X, int x_dtype, float* Y, int n_rows, int M, int K,
                            int epilogue, void* workspace, size_t ws_bytes, mxd_stream_t stream) {
    if (int rc = check_f16(W, X, Y, n_rows, M, K, "mxd_gemm_f16")) return rc;
    MXD_REQUIRE(epilogue == MXD_EPI_STORE || epilogue == MXD_EPI_ADD, MXD_ERR_INVALID_ARG,
                "mxd_gemm_f16: epilogue %d (store or add)", epilogue);
    MXD_REQUIRE(x_dtype == MXD_F16 || x_dtype == MXD_F32, MXD_ERR_INVALID_ARG, "mxd_gemm_f16: x_dtype %d", x_dtype);
    const size_t xesz = x_dtype == MXD_F32 ? 4 : 2;
    if (!use_mfma(MXD_W_F16, n_rows, K)) {  // few rows or K % 128: one matvec per row (fp32 X rounded the same way)
        for (int b = 0; b < n_rows; ++b) {
            const void* xb = static_cast<const char*>(X) + (size_t)b * K * xesz;
            const int rc = x_dtype == MXD_F32
                               ? mxd::matvec_xr16(MXD_W_F16, W, nullptr, static_cast<const float*>(xb),
                                                  Y + (size_t)b * M, M, K, epilogue, mxd::as_stream(stream))
                               : mxd_matvec_f16(W, xb, MXD_F16, Y + (size_t)b * M, M, K, epilogue, nullptr, stream);
            if (rc) return rc;
        }
        return MXD_OK;
    }
    GemmArgs a{};
    a.W[0] = a.W[1] = reinterpret_cast<const int8_t*>(W);
    a.X = static_cast<const uint16_t*>(X);
    a.Xf = static_cast<const float*>(X);
    a.Y = Y;
    a.n_rows = n_rows;
    a.M = M;
    a.K = K;
    hipStream_t s = mxd::as_stream(stream);
    if (x_dtype == MXD_F32) {
        if (epilogue == MXD_EPI_ADD)
            return launch_gemm<MXD_W_F16, 1, MXD_EPI_ADD, true>(a, workspace, ws_bytes, s, "mxd_gemm_f16");
        return launch_gemm<MXD_W_F16, 1, MXD_EPI_STORE, true>(a, workspace, ws_bytes, s, "mxd_gemm_f16");
    }
    if (epilogue == MXD_EPI_ADD) return launch_gemm<MXD_W_F16, 1, MXD_EPI_ADD>(a, workspace, ws_bytes, s, "mxd_gemm_f16");
    return launch_gemm<MXD_W_F16, 1, MXD_EPI_STORE>(a, workspace, ws_bytes, s, "mxd_gemm_f16");
}

extern "C" int mxd_gemm_gate_up_f16(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* X, float* H, int n_rows,
                                    int F, int K, int act, void* workspace, size_t ws_bytes, mxd_stream_t stream) {
    if (int rc = check_f16(Wg, X, H, n_rows, F, K, "mxd_gemm_gate_up_f16")) return rc;
    if (int rc = check_f16(Wu, X, H, n_rows, F, K, "mxd_gemm_gate_up_f16")) return rc;
    MXD_REQUIRE(act == MXD_ACT_GELU_TANH || act == MXD_ACT_SILU, MXD_ERR_INVALID_ARG,
                "mxd_gemm_gate_up_f16: unknown activation %d", act);
    if (!use_mfma(MXD_W_F16, n_rows, K)) {
        for (int b = 0; b < n_rows; ++b) {
            if (int rc = mxd_matvec_gate_up(MXD_W_F16, Wg, nullptr, Wu, nullptr, X + (size_t)b * K, MXD_F16,
                                            H + (size_t)b * F, F, K, act, stream))
                return rc;
        }
        return MXD_OK;
    }
    GemmArgs a{};
    a.W[0] = reinterpret_cast<const int8_t*>(Wg);
    a.W[1] = reinterpret_cast<const int8_t*>(Wu);
    a.X = X;
    a.Y = H;
    a.n_rows = n_rows;
    a.M = F;
    a.K = K;
    hipStream_t s = mxd::as_stream(stream);
    if (act == MXD_ACT_SILU)
        return launch_gemm<MXD_W_F16, 2, MXD_ACT_SILU>(a, workspace, ws_bytes, s, "mxd_gemm_gate_up_f16");
    return launch_gemm<MXD_W_F16, 2, MXD_ACT_GELU_TANH>(a, workspace, ws_bytes, s, "mxd_gemm_gate_up_f16");
}

bool mxd::gemm_on_matrix_cores(int n_rows, int K) { return use_mfma(MXD_W_F16, n_rows, K); }

int mxd::gemm_gate_up_f16_h16(const uint16_t* Wg, const uint16_t* Wu, const uint16_t* X, uint16_t* H, int n_rows,
                              int F, int K, int act, void* workspace, size_t ws_bytes, hipStream_t s) {
    const char* fn = "gemm_gate_up_f16_h16";
    MXD_REQUIRE(Wg && Wu && X && H, MXD_ERR_INVALID_ARG, "%s: null pointer", fn);
    MXD_REQUIRE(act == MXD_ACT_GELU_TANH || act == MXD_ACT_SILU, MXD_ERR_INVALID_ARG, "%s: unknown activation %d", fn,
                act);
    MXD_REQUIRE(F > 0 && use_mfma(MXD_W_F16, n_rows, K), MXD_ERR_UNSUPPORTED,
                "%s: n_rows=%d K=%d is not a matrix-core product", fn, n_rows, K);
    GemmArgs a{};
    a.W[0] = reinterpret_cast<const int8_t*>(Wg);
    a.W[1] = reinterpret_cast<const int8_t*>(Wu);
    a.X = X;
    a.Yh = H;
    a.n_rows = n_rows;
    a.M = F;
    a.K = K;
    if (act == MXD_ACT_SILU) return launch_gemm<MXD_W_F16, 2, MXD_ACT_SILU>(a, workspace, ws_bytes, s, fn);
    return launch_gemm<MXD_W_F16, 2, MXD_ACT_GELU_TANH>(a, workspace, ws_bytes, s, fn);
}
