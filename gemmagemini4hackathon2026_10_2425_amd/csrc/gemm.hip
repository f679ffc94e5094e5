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
// Work layout (gfx950, v_mfma_f32_16x16x32_f16):
//  * a workgroup of 8 waves owns 128 weight rows (16 per wave; for the
//    gate/up pair 64 rows of each matrix) x 64 activation rows x one split of
//    K of at most 1024 (8 steps of 128 = 4 quantisation blocks);
//  * the split's whole 64 x <=1024 fp16 activation slice is loaded into LDS
//    once (rows padded by 16 bytes so the 16-byte MFMA-operand reads are
//    conflict-free); after that one barrier the waves never synchronise
//    again: each streams its own weight rows straight from HBM through a
//    register ring GM_PD steps ahead of the math;
//  * one MFMA per (block, 16 activation rows) with the activations as the A
//    operand and the weights as B, so each lane's four results share one
//    weight row and one scale: acc += s * mfma(x, q, 0);
//  * K is split across workgroups (as many splits as the LDS slice needs, and
//    enough workgroups to fill the GPU); the fp32 partials are added in a
//    fixed order by a second kernel that also applies the epilogue, so
//    results are deterministic.
#include "common.hpp"

namespace {

constexpr int GM_WAVES = 8;
constexpr int GM_THREADS = GM_WAVES * 64;
constexpr int GM_ROWS = 16 * GM_WAVES;  // weight rows per workgroup (over both matrices)
constexpr int GM_BATCH = 64;            // activation rows per workgroup
constexpr int GM_KC = 128;              // K per step (4 blocks)
constexpr int GM_SMAX = 8;              // steps per split (LDS slice of 64 x 1024 halfs)
constexpr int GM_XP = GM_SMAX * GM_KC + 8;  // LDS pitch in halfs (+16 bytes)

struct GemmArgs {
    const int8_t* W[2];
    const uint16_t* S[2];
    const uint16_t* X;  // fp16 [n_rows][K]
    float* Y;           // fp32 [n_rows][M]
    float* part;        // fp32 [splits][n_rows][NMAT][M] when splits > 1
    int n_rows, M, K, splits, ksteps;
};

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



// Weight steps kept in flight per lane (a register ring), and the per-wave
// LDS staging of one step's weights (16 rows of 128 bytes, rows padded by 16
// bytes: the 8-byte MFMA-operand reads are conflict-free) and of the split's
// scales (16 rows x up to 32 blocks).
constexpr int GM_PD = 4;
constexpr int GM_WP = GM_KC + 16;
constexpr size_t GM_LDS_X = (size_t)GM_BATCH * GM_XP * 2;
constexpr size_t GM_LDS_W = (size_t)GM_WAVES * 16 * GM_WP;
constexpr size_t GM_LDS_S = (size_t)GM_WAVES * 16 * GM_SMAX * 4 * 2;
constexpr size_t GM_LDS = GM_LDS_X + GM_LDS_W + GM_LDS_S;  // 155 KiB of the CU's 160

template <int NMAT, int OP>
__global__ void __launch_bounds__(GM_THREADS) gemm_q8_kernel(GemmArgs a) {
    constexpr int ROWS_PER_MAT = GM_ROWS / NMAT;       // 128 or 64
    constexpr int WAVES_PER_MAT = GM_WAVES / NMAT;     // 8 or 4
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    _Float16* xs = reinterpret_cast<_Float16*>(smem);  // [GM_BATCH][GM_XP]

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;
    unsigned char* wst = smem + GM_LDS_X + (size_t)wave * 16 * GM_WP;                          // [16][GM_WP]
    uint16_t* sst = reinterpret_cast<uint16_t*>(smem + GM_LDS_X + GM_LDS_W) + wave * 16 * GM_SMAX * 4;  // [16][32]
    const int m = wave / WAVES_PER_MAT;  // which matrix this wave reads
    // Grid (splits, row tiles, batch tiles): consecutive workgroups take the
    // consecutive K splits of one row tile, so the workgroups running at once
    // read whole contiguous stretches of the weight rows (HBM-page friendly).
    const int row0 = blockIdx.y * ROWS_PER_MAT + 16 * (wave % WAVES_PER_MAT);
    const int split = blockIdx.x, b0 = blockIdx.z * GM_BATCH;
    const int M = a.M, K = a.K;
    const int ks0 = split * a.ksteps / a.splits, ks1 = (split + 1) * a.ksteps / a.splits;  // <= GM_SMAX steps
    const int nst = ks1 - ks0;

    // Weights are read row-contiguously: load u of a step gives lane l the 16
    // bytes at 16 (l & 7) of row 8u + (l >> 3)'s 128-byte step segment, so each
    // load is 8 whole 128-byte lines. Rows past M are clamped (never stored).
    const int8_t* wbase[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        wbase[u] = a.W[m] + (size_t)min(row0 + 8 * u + (lane >> 3), M - 1) * K + (size_t)ks0 * GM_KC + 16 * (lane & 7);
    auto load_w = [&](u4_t (&st)[2], int t) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
            st[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(wbase[u] + (size_t)t * GM_KC));
    };
    u4_t w[GM_PD][2];
#pragma unroll
    for (int p = 0; p < GM_PD; ++p)
        if (p < nst) load_w(w[p], p);

    // The split's scales: lane (col, g) fetches the 4 scales of steps g and
    // g + 4 of its row col.
    {
        const uint16_t* srow = a.S[m] + (size_t)min(row0 + col, M - 1) * (K / 32) + (size_t)ks0 * 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = g + 4 * h;
            if (t < nst)
                *reinterpret_cast<u2_t*>(&sst[col * GM_SMAX * 4 + 4 * t]) = *reinterpret_cast<const u2_t*>(srow + 4 * t);
        }
    }

    // Activation slice: 64 rows x nst * 128 halfs in 16-byte pieces, rows past
    // n_rows zero. Thread t takes row t / 8 and pieces t % 8 + 8u (no integer
    // division); all its loads are issued before any store (from clamped,
    // always valid addresses), so their latencies overlap.
    {
        constexpr int TPR = GM_THREADS / GM_BATCH;           // threads per row (8)
        constexpr int NPT = GM_SMAX * (GM_KC / 8) / TPR;     // pieces per thread (16)
        const int per_row = nst * (GM_KC / 8);
        const int r = threadIdx.x / TPR, sub = threadIdx.x % TPR;
        const uint16_t* xrow = a.X + (size_t)min(b0 + r, a.n_rows - 1) * K + (size_t)ks0 * GM_KC;
        u4_t v[NPT];
#pragma unroll
        for (int u = 0; u < NPT; ++u) {
            const int piece = min(sub + TPR * u, per_row - 1);
            v[u] = *reinterpret_cast<const u4_t*>(xrow + piece * 8);
        }
        const bool live = b0 + r < a.n_rows;
#pragma unroll
        for (int u = 0; u < NPT; ++u) {
            const int piece = sub + TPR * u;
            if (piece < per_row) {
                const u4_t z = {0u, 0u, 0u, 0u};
                *reinterpret_cast<u4_t*>(&xs[r * GM_XP + piece * 8]) = live ? v[u] : z;
            }
        }
    }
    __syncthreads();

    f4_t acc[4];
#pragma unroll
    for (int bg = 0; bg < 4; ++bg) acc[bg] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const f4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb = 0; kb < nst; kb += GM_PD) {
#pragma unroll
        for (int p = 0; p < GM_PD; ++p) {
            const int t = kb + p;  // step within the split
            if (t < nst) {
                // The step's weights through this wave's LDS slab into MFMA
                // operand order (only this wave touches the slab: LDS accesses
                // of one wave are ordered, the wave barrier orders the code).
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    *reinterpret_cast<u4_t*>(wst + (8 * u + (lane >> 3)) * GM_WP + 16 * (lane & 7)) = w[p][u];
                if (t + GM_PD < nst) load_w(w[p], t + GM_PD);
                __builtin_amdgcn_wave_barrier();
                // All operands of the step first, then the 16 independent
                // MFMAs back to back, then the per-block scaling, so no MFMA
                // result is waited for while the matrix core could be busy.
                h8_t wop[4];
                float sc[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u2_t q = *reinterpret_cast<const u2_t*>(wst + col * GM_WP + 32 * j + 8 * g);
                    h2_t h[4];
                    mxd::i8x4_to_h2x2(q.x, h[0], h[1]);
                    mxd::i8x4_to_h2x2(q.y, h[2], h[3]);
                    wop[j] = h8_t{h[0].x, h[0].y, h[1].x, h[1].y, h[2].x, h[2].y, h[3].x, h[3].y};
                    sc[j] = mxd::h2f(sst[col * GM_SMAX * 4 + 4 * t + j]);
                }
                h8_t xop[4][4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int bg = 0; bg < 4; ++bg)
                        xop[j][bg] = *reinterpret_cast<const h8_t*>(
                            &xs[(bg * 16 + col) * GM_XP + t * GM_KC + 32 * j + 8 * g]);
                f4_t c[4][4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int bg = 0; bg < 4; ++bg)
                        c[j][bg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop[j][bg], wop[j], zero, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int bg = 0; bg < 4; ++bg)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[bg][i] = fmaf(sc[j], c[j][bg][i], acc[bg][i]);
                __builtin_amdgcn_wave_barrier();
            }
        }
    }

    // Lane (col, g) holds rows b0 + 16 bg + 4 g + i of weight row row0 + col.
    const int wr = row0 + col;
    if (a.splits > 1) {
        if (wr < M) {
#pragma unroll
            for (int bg = 0; bg < 4; ++bg)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int b = b0 + 16 * bg + 4 * g + i;
                    if (b < a.n_rows) a.part[(((size_t)split * a.n_rows + b) * NMAT + m) * M + wr] = acc[bg][i];
                }
        }
        return;
    }
    if constexpr (NMAT == 2) {
        // The up waves hand their sums to the gate waves holding the same rows
        // through LDS (the activation slice is no longer needed).
        float* xf = reinterpret_cast<float*>(smem);
        __syncthreads();
        if (m == 1) {
#pragma unroll
            for (int bg = 0; bg < 4; ++bg)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xf[(((wave - WAVES_PER_MAT) * 4 + bg) * 4 + i) * 64 + lane] = acc[bg][i];
        }
        __syncthreads();
        if (m == 1 || wr >= M) return;
#pragma unroll
        for (int bg = 0; bg < 4; ++bg)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int b = b0 + 16 * bg + 4 * g + i;
                const float u = xf[((wave * 4 + bg) * 4 + i) * 64 + lane];
                if (b < a.n_rows) a.Y[(size_t)b * M + wr] = epilogue<NMAT, OP>(acc[bg][i], u, 0.0f);
            }
    } else {
        if (wr >= M) return;
#pragma unroll
        for (int bg = 0; bg < 4; ++bg)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int b = b0 + 16 * bg + 4 * g + i;
                if (b < a.n_rows) {
                    float* y = a.Y + (size_t)b * M + wr;
                    *y = epilogue<NMAT, OP>(acc[bg][i], 0.0f, OP == MXD_EPI_ADD ? *y : 0.0f);
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
        a.Y[e] = epilogue<NMAT, OP>(s0, s1, OP == MXD_EPI_ADD && NMAT == 1 ? a.Y[e] : 0.0f);
    }
}

bool use_mfma(int n_rows, int K) {
    return n_rows >= mxd::tunable("GM_MIN_ROWS", 16) && K % GM_KC == 0;
}

// K splits: at least enough that a split's activation slice fits the LDS
// (GM_SMAX steps), and enough workgroups for one per CU; the GM_SPLITS tunable
// can ask for more (up to one step per split), never fewer.
int pick_splits(int n_rows, int M, int K, int nmat) {
    const int tiles = ((M + GM_ROWS / nmat - 1) / (GM_ROWS / nmat)) * ((n_rows + GM_BATCH - 1) / GM_BATCH);
    const int ksteps = K / GM_KC;
    const int min_s = (ksteps + GM_SMAX - 1) / GM_SMAX;
    int s = mxd::tunable("GM_SPLITS", max(min_s, (256 + tiles - 1) / tiles));
    return max(min_s, min(s, ksteps));
}

size_t ws_bytes_for(int n_rows, int M, int K, int nmat) {
    if (n_rows <= 0 || M <= 0 || K <= 0 || !use_mfma(n_rows, K)) return 0;
    const int s = pick_splits(n_rows, M, K, nmat);
    return s > 1 ? (size_t)s * n_rows * nmat * M * sizeof(float) : 0;
}

template <int NMAT, int OP>
int launch_gemm(GemmArgs a, void* ws, size_t ws_bytes, hipStream_t s, const char* fn) {
    a.ksteps = a.K / GM_KC;
    a.splits = pick_splits(a.n_rows, a.M, a.K, NMAT);
    const size_t need = a.splits > 1 ? (size_t)a.splits * a.n_rows * NMAT * a.M * sizeof(float) : 0;
    MXD_REQUIRE(need == 0 || (ws && ws_bytes >= need), MXD_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)",
                fn, need, ws_bytes);
    a.part = static_cast<float*>(ws);
    const dim3 grid(a.splits, (a.M + GM_ROWS / NMAT - 1) / (GM_ROWS / NMAT), (a.n_rows + GM_BATCH - 1) / GM_BATCH);
    const size_t lds = GM_LDS;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_q8_kernel<NMAT, OP>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    MXD_REQUIRE(attr == hipSuccess, MXD_ERR_HIP, "%s: cannot enable %zu bytes of LDS: %s", fn, lds,
                hipGetErrorString(attr));
    hipLaunchKernelGGL((gemm_q8_kernel<NMAT, OP>), grid, dim3(GM_THREADS), lds, s, a);
    if (a.splits > 1) {
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

extern "C" size_t mxd_gemm_q8b32_workspace_size(int n_rows, int M, int K) { return ws_bytes_for(n_rows, M, K, 1); }

extern "C" size_t mxd_gemm_gate_up_q8b32_workspace_size(int n_rows, int F, int K) {
    return ws_bytes_for(n_rows, F, K, 2);
}

extern "C" int mxd_gemm_q8b32(const int8_t* Wq, const uint16_t* scales, const uint16_t* X, float* Y, int n_rows, int M,
                              int K, int epilogue, void* workspace, size_t ws_bytes, mxd_stream_t stream) {
    if (int rc = check_common(Wq, scales, X, Y, n_rows, M, K, "mxd_gemm_q8b32")) return rc;
    MXD_REQUIRE(epilogue == MXD_EPI_STORE || epilogue == MXD_EPI_ADD, MXD_ERR_INVALID_ARG,
                "mxd_gemm_q8b32: epilogue %d (store or add)", epilogue);
    if (!use_mfma(n_rows, K)) {  // few rows: one matvec per row
        for (int b = 0; b < n_rows; ++b) {
            if (int rc = mxd_matvec_q8b32(Wq, scales, X + (size_t)b * K, MXD_F16, Y + (size_t)b * M, M, K, epilogue,
                                          nullptr, stream))
                return rc;
        }
        return MXD_OK;
    }
    GemmArgs a{};
    a.W[0] = a.W[1] = Wq;
    a.S[0] = a.S[1] = scales;
    a.X = X;
    a.Y = Y;
    a.n_rows = n_rows;
    a.M = M;
    a.K = K;
    hipStream_t s = mxd::as_stream(stream);
    if (epilogue == MXD_EPI_ADD) return launch_gemm<1, MXD_EPI_ADD>(a, workspace, ws_bytes, s, "mxd_gemm_q8b32");
    return launch_gemm<1, MXD_EPI_STORE>(a, workspace, ws_bytes, s, "mxd_gemm_q8b32");
}

extern "C" int mxd_gemm_gate_up_q8b32(const int8_t* Wg, const uint16_t* sg, const int8_t* Wu, const uint16_t* su,
                                      const uint16_t* X, float* H, int n_rows, int F, int K, int act, void* workspace,
                                      size_t ws_bytes, mxd_stream_t stream) {
    if (int rc = check_common(Wg, sg, X, H, n_rows, F, K, "mxd_gemm_gate_up_q8b32")) return rc;
    if (int rc = check_common(Wu, su, X, H, n_rows, F, K, "mxd_gemm_gate_up_q8b32")) return rc;
    MXD_REQUIRE(act == MXD_ACT_GELU_TANH || act == MXD_ACT_SILU, MXD_ERR_INVALID_ARG,
                "mxd_gemm_gate_up_q8b32: unknown activation %d", act);
    if (!use_mfma(n_rows, K)) {
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
        return launch_gemm<2, MXD_ACT_SILU>(a, workspace, ws_bytes, s, "mxd_gemm_gate_up_q8b32");
    return launch_gemm<2, MXD_ACT_GELU_TANH>(a, workspace, ws_bytes, s, "mxd_gemm_gate_up_q8b32");
}
