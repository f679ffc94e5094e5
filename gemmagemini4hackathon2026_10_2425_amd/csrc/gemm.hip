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
//  * a workgroup of 4 waves owns 64 weight rows (16 per wave; for the
//    gate/up pair 32 rows of each matrix) x 64 activation rows x one split of K;
//  * K advances in steps of 128 (4 quantisation blocks): the 64 x 128 fp16
//    activation tile is staged in LDS once per workgroup (rows padded by
//    16 bytes so the 16-byte MFMA-operand reads are conflict-free) while every
//    wave streams its own weight rows straight from HBM into registers, one
//    step ahead of the math;
//  * one MFMA per (block, 16 activation rows) with the activations as the A
//    operand and the weights as B, so each lane's four results share one
//    weight row and one scale: acc += s * mfma(x, q, 0);
//  * small weight matrices split K across workgroups to fill the GPU; the
//    fp32 partials are added in a fixed order by a second kernel that also
//    applies the epilogue, so results are deterministic.
#include "common.hpp"

namespace {

constexpr int GM_THREADS = 256;  // 4 waves
constexpr int GM_ROWS = 64;      // weight rows per workgroup (over both matrices)
constexpr int GM_BATCH = 64;     // activation rows per workgroup
constexpr int GM_KC = 128;       // K per step (4 blocks)
constexpr int GM_XP = GM_KC + 8; // LDS pitch in halfs (+16 bytes)

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

// One K step of weights for one lane: 4 blocks x 8 int8 and the 4 scales.
struct WStep {
    u2_t q[4];
    u2_t s;
};

template <int NMAT, int OP>
__global__ void __launch_bounds__(GM_THREADS) gemm_q8_kernel(GemmArgs a) {
    constexpr int ROWS_PER_MAT = GM_ROWS / NMAT;      // 64 or 32
    constexpr int WAVES_PER_MAT = 4 / NMAT;           // 4 or 2
    __shared__ __attribute__((aligned(16))) _Float16 xs[GM_BATCH * GM_XP];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int m = wave / WAVES_PER_MAT;  // which matrix this wave reads
    const int row0 = blockIdx.x * ROWS_PER_MAT + 16 * (wave % WAVES_PER_MAT);
    const int split = blockIdx.y, b0 = blockIdx.z * GM_BATCH;
    const int M = a.M, K = a.K;
    const int ks0 = split * a.ksteps / a.splits, ks1 = (split + 1) * a.ksteps / a.splits;

    // This lane's weight row (clamped: rows past M compute garbage that is
    // never stored) and its scale row.
    const int wrow = min(row0 + col, M - 1);
    const int8_t* wq = a.W[m] + (size_t)wrow * K + 8 * g;
    const uint16_t* ws = a.S[m] + (size_t)wrow * (K / 32);

    auto load_w = [&](WStep& st, int ks) {
        const int8_t* p = wq + (size_t)ks * GM_KC;
#pragma unroll
        for (int j = 0; j < 4; ++j) st.q[j] = __builtin_nontemporal_load(reinterpret_cast<const u2_t*>(p + 32 * j));
        st.s = *reinterpret_cast<const u2_t*>(ws + ks * 4);
    };

    f4_t acc[4];
#pragma unroll
    for (int bg = 0; bg < 4; ++bg) acc[bg] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    WStep cur, nxt;
    if (ks0 < ks1) load_w(cur, ks0);
    for (int ks = ks0; ks < ks1; ++ks) {
        if (ks + 1 < ks1) load_w(nxt, ks + 1);
        // Stage the 64 x 128 activation tile: 1024 16-byte pieces, 4 per thread.
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = threadIdx.x + GM_THREADS * u;
            const int r = idx >> 4, seg = idx & 15;
            u4_t v = {0u, 0u, 0u, 0u};
            if (b0 + r < a.n_rows)
                v = *reinterpret_cast<const u4_t*>(a.X + (size_t)(b0 + r) * K + (size_t)ks * GM_KC + seg * 8);
            *reinterpret_cast<u4_t*>(&xs[r * GM_XP + seg * 8]) = v;
        }
        __syncthreads();
        const f4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h2_t h[4];
            mxd::i8x4_to_h2x2(cur.q[j].x, h[0], h[1]);
            mxd::i8x4_to_h2x2(cur.q[j].y, h[2], h[3]);
            const h8_t wop = {h[0].x, h[0].y, h[1].x, h[1].y, h[2].x, h[2].y, h[3].x, h[3].y};
            const uint16_t sb = (uint16_t)((j & 1) ? (cur.s[j >> 1] >> 16) : (cur.s[j >> 1] & 0xFFFFu));
            const float sc = mxd::h2f(sb);
#pragma unroll
            for (int bg = 0; bg < 4; ++bg) {
                const h8_t xop = *reinterpret_cast<const h8_t*>(&xs[(bg * 16 + col) * GM_XP + 32 * j + 8 * g]);
                const f4_t c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop, wop, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[bg][i] = fmaf(sc, c[i], acc[bg][i]);
            }
        }
        __syncthreads();  // the tile is rewritten next step
        cur = nxt;
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
        // The up waves (2, 3) hand their sums to the gate waves (0, 1) holding
        // the same rows through LDS (the activation tile is no longer needed).
        float* xf = reinterpret_cast<float*>(xs);
        if (m == 1) {
#pragma unroll
            for (int bg = 0; bg < 4; ++bg)
#pragma unroll
                for (int i = 0; i < 4; ++i) xf[(((wave - 2) * 4 + bg) * 4 + i) * 64 + lane] = acc[bg][i];
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

// K splits: enough workgroups for about two per CU, at least one K step each.
int pick_splits(int n_rows, int M, int K, int nmat) {
    const int tiles = ((M + GM_ROWS / nmat - 1) / (GM_ROWS / nmat)) * ((n_rows + GM_BATCH - 1) / GM_BATCH);
    const int ksteps = K / GM_KC;
    int s = mxd::tunable("GM_SPLITS", max(1, 512 / tiles));
    return max(1, min(s, ksteps));
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
    const dim3 grid((a.M + GM_ROWS / NMAT - 1) / (GM_ROWS / NMAT), a.splits, (a.n_rows + GM_BATCH - 1) / GM_BATCH);
    hipLaunchKernelGGL((gemm_q8_kernel<NMAT, OP>), grid, dim3(GM_THREADS), 0, s, a);
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
