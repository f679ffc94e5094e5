// Matrix-vector products for single-token decode: fp32, fp16 and int8
// block-32 weights, with store / residual-add / gelu*aux epilogues and the
// fused gate-up (GLU) variant.
//
// Layout of the work (gfx950): a workgroup owns NR consecutive output rows and
// NW wavefronts. The K axis is cut into chunks of 64 lanes x 16 bytes (one
// coalesced 1 KiB wave load per row); wave w takes chunks w, w+NW, ... so the
// NW waves of a workgroup stream adjacent KiBs of the same rows. Each wave keeps
// U chunks x NR rows (x NMAT matrices) of loads in flight before doing any
// math, reduces with DPP + bpermute, and the NW partial sums of a row are added
// in a fixed order through LDS, so results are deterministic run to run.
//
// Reference semantics: matvec_f16 / matvec_gate_up_* (KG/kernels.metal:159-234,
// KL/kernels.metal:106-173): fp32 accumulation of float(w) * x.
#include <type_traits>

#include "gemv_core.hpp"

namespace {

// NMAT == 1: OP is an MXD_EPI_* or EPI_ROPE_KV; NMAT == 2: OP is an MXD_ACT_*
// (gate, up).
template <int WF, typename XT, int NMAT, int OP, int NR, int NW, bool RES = false>
__global__ void __launch_bounds__(NW * 64) gemv_kernel(GemvArgs a) {
    if constexpr (RES) residual_prologue<NW>(a);
    constexpr int EPL = WT<WF>::EPL;
    constexpr int CH = 64 * EPL;
    constexpr int U = (8 / (NR * NMAT)) > 0 ? (8 / (NR * NMAT)) : 1;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * NR;
    const int M = a.M, K = a.K;
    const int nch = (K + CH - 1) / CH;

    const unsigned char* wrow[NMAT][NR];
    const uint16_t* srow[NMAT][NR];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            int row = min(r0 + r, M - 1);
            if constexpr (OP == EPI_ROPE_KV) row = rope_row(row, a);
            wrow[m][r] = static_cast<const unsigned char*>(a.W[m]) + (size_t)row * K * welem_bytes<WF>();
            srow[m][r] = WF == MXD_W_Q8B32 ? a.S[m] + (size_t)row * (K / 32) : nullptr;
        }

    float acc[NMAT][NR];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[m][r] = 0.0f;

    // Fused RMSNorm: the loop accumulates w . (x * w_norm) and the row sums are
    // scaled by rsqrt(mean(x^2) + eps) at the end, so the norm's reduction runs
    // after the weight stream instead of delaying its first loads.
    for (int c0 = wave; c0 < nch; c0 += NW * U) {
        u4_t wv[U][NMAT][NR];
        uint16_t sv[U][NMAT][NR];
        XFrag<XT, EPL> xf[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * NW;
            const int col = c * CH + lane * EPL;
            ok[u] = (c < nch) && (col < K);
            if (ok[u]) {
                if (a.mpo)
                    xf[u].load_merge(a, col);
                else if (a.nw)
                    xf[u].load_norm(a.x, a.nw, col, 1.0f, a.plus_one);
                else
                    xf[u].load(a.x, col, a.xr16);
#pragma unroll
                for (int m = 0; m < NMAT; ++m)
#pragma unroll
                    for (int r = 0; r < NR; ++r) {
                        wv[u][m][r] = ld_stream<WF>(wrow[m][r] + (size_t)col * welem_bytes<WF>());
                        if (WF == MXD_W_Q8B32) sv[u][m][r] = srow[m][r][col / 32];
                    }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    if constexpr (WF == MXD_W_Q8B32)
                        acc[m][r] = fmaf(dot16q(wv[u][m][r], xf[u]), mxd::h2f(sv[u][m][r]), acc[m][r]);
                    else
                        acc[m][r] = dot16(wv[u][m][r], xf[u], acc[m][r]);
                }
        }
    }

    const float nscale = a.nw ? block_rms_scale<NW>(static_cast<const float*>(a.x), K, a.eps) : 1.0f;
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[m][r] = mxd::wave_sum(acc[m][r]);

    if constexpr (NW > 1) {
        __shared__ float red[NW][NMAT][NR];
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int r = 0; r < NR; ++r) red[wave][m][r] = acc[m][r];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                float s = red[0][m][r];
#pragma unroll
                for (int w = 1; w < NW; ++w) s += red[w][m][r];
                acc[m][r] = s;
            }
    }
    if (a.nw) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[m][r] *= nscale;
    }

    if constexpr (OP == EPI_ROPE_KV) {
        // Rotate each (i, i + hd/2) pair at pos (angle pos * inv_freq[i] in fp32,
        // accurate sin/cos) and write q to y, k and v (fp16) to the tiled caches
        // (KL/kernels.metal:199-222).
        if (lane == 0) {
            const int pos = a.pos_dev ? a.pos_dev[0] : a.pos;
            const int half = a.hd >> 1, qk_rows = (a.n_heads + a.n_kv) * a.hd;
            const bool in_cache = pos >= 0 && pos < a.max_ctx;
            const int kpos = pos & 31;
#pragma unroll
            for (int r = 0; r < NR; r += 2) {
                const int v = r0 + r;
                if (v >= M) break;
                if (v < qk_rows) {
                    const int p = v >> 1, head = p / half, i = p - head * half;
                    const float ang = (float)pos * a.inv_freq[i];
                    float sn, cs;
                    sincosf(ang, &sn, &cs);
                    const float x0 = acc[0][r], x1 = acc[0][r + 1];
                    const float ra = x0 * cs - x1 * sn;
                    const float rb = x1 * cs + x0 * sn;
                    if (head < a.n_heads) {
                        a.y[head * a.hd + i] = ra;
                        a.y[head * a.hd + i + half] = rb;
                    } else if (in_cache) {
                        const size_t tile = ((size_t)(head - a.n_heads) * a.max_ctx + (pos & ~31)) * a.hd;
                        a.kcache[tile + mxd::k_tile_offset(kpos, i, a.hd)] = mxd::f2h_bits(ra);
                        a.kcache[tile + mxd::k_tile_offset(kpos, i + half, a.hd)] = mxd::f2h_bits(rb);
                    }
                } else if (in_cache) {
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        if (v + e >= M) break;
                        const int vr = v + e - qk_rows, kvh = vr / a.hd, d = vr - kvh * a.hd;
                        const size_t tile = ((size_t)kvh * a.max_ctx + (pos & ~31)) * a.hd;
                        a.vcache[tile + mxd::v_tile_offset(kpos, d)] = mxd::f2h_bits(acc[0][r + e]);
                    }
                }
            }
        }
        return;
    }

    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int row = r0 + r;
            if (row >= M) break;
            if constexpr (NMAT == 2) {
                const float g = acc[0][r], u = acc[1][r];
                a.y[row] = (OP == MXD_ACT_SILU ? mxd::silu(g) : mxd::gelu_tanh(g)) * u;
            } else if constexpr (OP == MXD_EPI_ADD) {
                a.y[row] += acc[0][r];
            } else if constexpr (OP == MXD_EPI_GELU_MUL) {
                a.y[row] = mxd::gelu_tanh(acc[0][r]) * a.aux[row];
            } else {
                a.y[row] = acc[0][r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row-streaming variant. A persistent grid walks the rows front to back
// (workgroup b takes rows b, b + grid, ...); the NW waves of a workgroup split
// one row's chunks (wave w always owns chunks w, w + NW, ... of every row), so
// at any moment the whole GPU reads one compact, sequential window of W, which
// is what keeps the HBM pages open. Each wave keeps its x fragments in
// registers for the whole kernel, streams W with nontemporal loads (W is read
// once), and issues the next row's loads before reducing the current row.
// The NW partial sums of a row are added in a fixed order (deterministic).
// ---------------------------------------------------------------------------
constexpr int RS_MAX_CHUNKS = 64;  // 16 waves x 4 chunks

// Dynamic LDS of a launch: the residual prologue's x' (K floats).
size_t dyn_lds(const GemvArgs& a) { return a.rsrc ? (size_t)a.K * sizeof(float) : 0; }

template <int WF, typename XT, int NMAT, int OP, int NW, int RS_CPW, bool RES = false>
__global__ void __launch_bounds__(NW * 64) gemv_rows_kernel(GemvArgs a) {
    constexpr int EPL = WT<WF>::EPL;
    constexpr int CH = 64 * EPL;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int M = a.M, K = a.K;
    const int nch = (K + CH - 1) / CH;
    const size_t row_bytes = (size_t)K * welem_bytes<WF>();

    // This wave's columns: chunk wave + j * NW for j < RS_CPW (the host picks
    // RS_CPW = ceil(nch / NW)).
    int col[RS_CPW];
    bool ok[RS_CPW];
    XFrag<XT, EPL> xf[RS_CPW];
#pragma unroll
    for (int j = 0; j < RS_CPW; ++j) {
        col[j] = (wave + j * NW) * CH + lane * EPL;
        ok[j] = (wave + j * NW) < nch && col[j] < K;
    }

    __shared__ float red[2][NW][NMAT];
    u4_t wv[RS_CPW][NMAT];
    uint16_t sv[RS_CPW][NMAT];
    auto issue = [&](int row) {
#pragma unroll
        for (int j = 0; j < RS_CPW; ++j)
            if (ok[j]) {
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    const unsigned char* base = static_cast<const unsigned char*>(a.W[m]) + (size_t)row * row_bytes;
                    wv[j][m] = ld_stream<WF>(base + (size_t)col[j] * welem_bytes<WF>());
                    if (WF == MXD_W_Q8B32) sv[j][m] = a.S[m][(size_t)row * (K / 32) + col[j] / 32];
                }
            }
    };

    auto load_x = [&]() {
        const float nscale = a.nw ? block_rms_scale<NW>(static_cast<const float*>(a.x), K, a.eps) : 1.0f;
#pragma unroll
        for (int j = 0; j < RS_CPW; ++j) {
            if (ok[j]) {
                if (a.nw)
                    xf[j].load_norm(a.x, a.nw, col[j], nscale, a.plus_one);
                else
                    xf[j].load(a.x, col[j], a.xr16);
            }
        }
    };
    int row = blockIdx.x;
    if constexpr (RES) {
        // the first row's weights in flight before the prologue's round trip
        if (row < M) issue(row);
        residual_prologue<NW>(a);
        load_x();
    } else {
        load_x();
        if (row < M) issue(row);
    }
    int buf = 0;
    for (; row < M; row += gridDim.x) {
        float acc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < RS_CPW; ++j)
            if (ok[j]) {
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    if constexpr (WF == MXD_W_Q8B32)
                        acc[m] = fmaf(dot16q(wv[j][m], xf[j]), mxd::h2f(sv[j][m]), acc[m]);
                    else
                        acc[m] = dot16(wv[j][m], xf[j], acc[m]);
                }
            }
        const int next = row + gridDim.x;
        if (next < M) issue(next);  // the next row streams in while this one reduces
#pragma unroll
        for (int m = 0; m < NMAT; ++m) acc[m] = mxd::wave_sum(acc[m]);
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m) red[buf][wave][m] = acc[m];
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float s[NMAT];
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                s[m] = red[buf][0][m];
#pragma unroll
                for (int w = 1; w < NW; ++w) s[m] += red[buf][w][m];
            }
            if constexpr (NMAT == 2) {
                a.y[row] = (OP == MXD_ACT_SILU ? mxd::silu(s[0]) : mxd::gelu_tanh(s[0])) * s[1];
            } else if constexpr (OP == MXD_EPI_ADD) {
                a.y[row] += s[0];
            } else if constexpr (OP == MXD_EPI_GELU_MUL) {
                a.y[row] = mxd::gelu_tanh(s[0]) * a.aux[row];
            } else {
                a.y[row] = s[0];
            }
        }
        buf ^= 1;
    }
}

// Whether a launch takes the residual prologue (fp16 weights, fp32 x only:
// the kernels without it keep their x in the global address space).
template <int WF, typename XT, int OP>
constexpr bool res_capable() {
    return WF == MXD_W_F16 && std::is_same<XT, float>::value && OP != EPI_ROPE_KV;
}

template <int WF, typename XT, int NMAT, int OP, int NW, int CPW, bool RES>
int launch_rows_kr(const GemvArgs& a, int wg_per_cu, hipStream_t s) {
    auto kern = gemv_rows_kernel<WF, XT, NMAT, OP, NW, CPW, RES>;
    // A persistent grid must fit on the GPU at once: cap by the occupancy the
    // kernel's registers and LDS allow.
    const size_t dyn = dyn_lds(a);
    int fit = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&fit, kern, NW * 64, dyn) != hipSuccess || fit < 1) fit = 1;
    if (wg_per_cu > fit) wg_per_cu = fit;
    int grid = 256 * wg_per_cu;
    if (grid > a.M) grid = a.M;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), dyn, s, a);
    return mxd::check_launch("matvec");
}

template <int WF, typename XT, int NMAT, int OP, int NW, int CPW>
int launch_rows_k(const GemvArgs& a, int wg_per_cu, hipStream_t s) {
    if constexpr (res_capable<WF, XT, OP>()) {
        if (a.rsrc) return launch_rows_kr<WF, XT, NMAT, OP, NW, CPW, true>(a, wg_per_cu, s);
    }
    return launch_rows_kr<WF, XT, NMAT, OP, NW, CPW, false>(a, wg_per_cu, s);
}

template <int WF, typename XT, int NMAT, int OP>
int launch_rows(const GemvArgs& a, int nw, int cpw, int wg_per_cu, hipStream_t s) {
    if (nw == 4 && cpw == 1) return launch_rows_k<WF, XT, NMAT, OP, 4, 1>(a, wg_per_cu, s);
    if (nw == 4 && cpw == 2) return launch_rows_k<WF, XT, NMAT, OP, 4, 2>(a, wg_per_cu, s);
    if (nw == 4 && cpw == 4) return launch_rows_k<WF, XT, NMAT, OP, 4, 4>(a, wg_per_cu, s);
    if (nw == 8 && cpw == 1) return launch_rows_k<WF, XT, NMAT, OP, 8, 1>(a, wg_per_cu, s);
    if (nw == 8 && cpw == 2) return launch_rows_k<WF, XT, NMAT, OP, 8, 2>(a, wg_per_cu, s);
    if (nw == 8 && cpw == 4) return launch_rows_k<WF, XT, NMAT, OP, 8, 4>(a, wg_per_cu, s);
    if (nw == 14 && cpw == 1) return launch_rows_k<WF, XT, NMAT, OP, 14, 1>(a, wg_per_cu, s);
    if (nw == 14 && cpw == 2) return launch_rows_k<WF, XT, NMAT, OP, 14, 2>(a, wg_per_cu, s);
    if (nw == 16 && cpw == 1) return launch_rows_k<WF, XT, NMAT, OP, 16, 1>(a, wg_per_cu, s);
    if (nw == 16 && cpw == 2) return launch_rows_k<WF, XT, NMAT, OP, 16, 2>(a, wg_per_cu, s);
    if (nw == 16 && cpw == 4) return launch_rows_k<WF, XT, NMAT, OP, 16, 4>(a, wg_per_cu, s);
    return mxd::fail(MXD_ERR_INVALID_ARG, "matvec: row streaming has no (waves %d, chunks/wave %d) variant", nw, cpw);
}

// ---------------------------------------------------------------------------
// Sweep variant. Workgroup b of a grid of G owns rows b, b + G, b + 2G, ...,
// and wave w owns chunks w, w + NW, ... (CPW of them) of each of those rows,
// so its x fragments stay in registers and at any moment the whole grid reads
// one compact window of W that moves front to back (the access pattern of a
// plain grid-stride read, the fastest way to stream HBM here). A wave keeps
// the next row's loads in flight while it reduces the current row; its
// per-row partial sums go to LDS slots (no barrier per row) and are added in
// a fixed order once at the end, so results are deterministic.
// ---------------------------------------------------------------------------
constexpr int SW_MAX_ROWS = 256;

template <int WF, typename XT, int NMAT, int OP, int NW, int CPW, bool RES = false>
__global__ void __launch_bounds__(NW * 64) gemv_sweep_kernel(GemvArgs a) {
    constexpr int EPL = WT<WF>::EPL;
    constexpr int CH = 64 * EPL;
    __shared__ float part[SW_MAX_ROWS][NMAT][NW];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int M = a.M, K = a.K, G = gridDim.x, b = blockIdx.x;
    const int nch = (K + CH - 1) / CH;
    const int nrows = b < M ? (M - b + G - 1) / G : 0;  // <= SW_MAX_ROWS (host)
    const size_t row_bytes = (size_t)K * welem_bytes<WF>();

    int col[CPW];
    bool ok[CPW];
    XFrag<XT, EPL> xf[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        col[j] = (wave + j * NW) * CH + lane * EPL;
        ok[j] = (wave + j * NW) < nch && col[j] < K;
    }
    auto load_x = [&]() {
#pragma unroll
        for (int j = 0; j < CPW; ++j)
            if (ok[j]) {
                if (a.nw)
                    xf[j].load_norm(a.x, a.nw, col[j], 1.0f, a.plus_one);
                else
                    xf[j].load(a.x, col[j], a.xr16);
            }
    };

    auto issue = [&](u4_t (&wv)[CPW][NMAT], uint16_t (&sv)[CPW][NMAT], int row) {
#pragma unroll
        for (int j = 0; j < CPW; ++j)
            if (ok[j]) {
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    const unsigned char* base = static_cast<const unsigned char*>(a.W[m]) + (size_t)row * row_bytes;
                    wv[j][m] = ld_stream<WF>(base + (size_t)col[j] * welem_bytes<WF>());
                    if (WF == MXD_W_Q8B32) sv[j][m] = a.S[m][(size_t)row * (K / 32) + col[j] / 32];
                }
            }
    };
    auto consume = [&](const u4_t (&wv)[CPW][NMAT], const uint16_t (&sv)[CPW][NMAT], int i) {
        float acc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPW; ++j)
            if (ok[j]) {
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    if constexpr (WF == MXD_W_Q8B32)
                        acc[m] = fmaf(dot16q(wv[j][m], xf[j]), mxd::h2f(sv[j][m]), acc[m]);
                    else
                        acc[m] = dot16(wv[j][m], xf[j], acc[m]);
                }
            }
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            acc[m] = mxd::wave_sum(acc[m]);
            if (lane == 0) part[i][m][wave] = acc[m];
        }
    };

    u4_t wa[CPW][NMAT], wb[CPW][NMAT];
    uint16_t sa[CPW][NMAT], sb[CPW][NMAT];
    if constexpr (RES) {
        // the first row's weights in flight before the prologue's round trip
        if (nrows > 0) issue(wa, sa, b);
        residual_prologue<NW>(a);
        load_x();
    } else {
        load_x();
        if (nrows > 0) issue(wa, sa, b);
    }
    for (int i = 0; i < nrows; i += 2) {
        if (i + 1 < nrows) issue(wb, sb, b + (i + 1) * G);
        consume(wa, sa, i);
        if (i + 1 >= nrows) break;
        if (i + 2 < nrows) issue(wa, sa, b + (i + 2) * G);
        consume(wb, sb, i + 1);
    }

    const float nscale = a.nw ? block_rms_scale<NW>(static_cast<const float*>(a.x), K, a.eps) : 1.0f;
    __syncthreads();
    for (int i = threadIdx.x; i < nrows; i += NW * 64) {
        const int row = b + i * G;
        float v[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            float t = part[i][m][0];
#pragma unroll
            for (int w = 1; w < NW; ++w) t += part[i][m][w];
            v[m] = a.nw ? t * nscale : t;
        }
        if constexpr (NMAT == 2) {
            a.y[row] = (OP == MXD_ACT_SILU ? mxd::silu(v[0]) : mxd::gelu_tanh(v[0])) * v[1];
        } else if constexpr (OP == MXD_EPI_ADD) {
            a.y[row] += v[0];
        } else if constexpr (OP == MXD_EPI_GELU_MUL) {
            a.y[row] = mxd::gelu_tanh(v[0]) * a.aux[row];
        } else {
            a.y[row] = v[0];
        }
    }
}

template <int WF, typename XT, int NMAT, int OP, int NW, int CPW, bool RES>
int launch_sweep_kr(const GemvArgs& a, int wg_per_cu, hipStream_t s) {
    auto kern = gemv_sweep_kernel<WF, XT, NMAT, OP, NW, CPW, RES>;
    const size_t dyn = dyn_lds(a);
    int fit = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&fit, kern, NW * 64, dyn) != hipSuccess || fit < 1) fit = 1;
    if (wg_per_cu > fit) wg_per_cu = fit;
    int grid = 256 * wg_per_cu;
    const int min_grid = (a.M + SW_MAX_ROWS - 1) / SW_MAX_ROWS;  // LDS holds SW_MAX_ROWS rows per workgroup
    if (grid < min_grid) grid = min_grid;
    if (grid > a.M) grid = a.M;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), dyn, s, a);
    return mxd::check_launch("matvec");
}

template <int WF, typename XT, int NMAT, int OP, int NW, int CPW>
int launch_sweep_k(const GemvArgs& a, int wg_per_cu, hipStream_t s) {
    if constexpr (res_capable<WF, XT, OP>()) {
        if (a.rsrc) return launch_sweep_kr<WF, XT, NMAT, OP, NW, CPW, true>(a, wg_per_cu, s);
    }
    return launch_sweep_kr<WF, XT, NMAT, OP, NW, CPW, false>(a, wg_per_cu, s);
}

template <int WF, typename XT, int NMAT, int OP>
int launch_sweep(const GemvArgs& a, int nw, int cpw, int wg_per_cu, hipStream_t s) {
    if (nw == 4 && cpw == 1) return launch_sweep_k<WF, XT, NMAT, OP, 4, 1>(a, wg_per_cu, s);
    if (nw == 4 && cpw == 2) return launch_sweep_k<WF, XT, NMAT, OP, 4, 2>(a, wg_per_cu, s);
    if (nw == 4 && cpw == 4) return launch_sweep_k<WF, XT, NMAT, OP, 4, 4>(a, wg_per_cu, s);
    if (nw == 8 && cpw == 1) return launch_sweep_k<WF, XT, NMAT, OP, 8, 1>(a, wg_per_cu, s);
    if (nw == 8 && cpw == 2) return launch_sweep_k<WF, XT, NMAT, OP, 8, 2>(a, wg_per_cu, s);
    if (nw == 8 && cpw == 4) return launch_sweep_k<WF, XT, NMAT, OP, 8, 4>(a, wg_per_cu, s);
    if (nw == 16 && cpw == 1) return launch_sweep_k<WF, XT, NMAT, OP, 16, 1>(a, wg_per_cu, s);
    if (nw == 16 && cpw == 2) return launch_sweep_k<WF, XT, NMAT, OP, 16, 2>(a, wg_per_cu, s);
    if (nw == 16 && cpw == 4) return launch_sweep_k<WF, XT, NMAT, OP, 16, 4>(a, wg_per_cu, s);
    return mxd::fail(MXD_ERR_INVALID_ARG, "matvec: sweep has no (waves %d, chunks/wave %d) variant", nw, cpw);
}

// Rows per workgroup and waves per workgroup for a shape, overridable through
// the MV_NR / MV_NW tunables. From sweeps on MI355X (117 MB to 1 GB matrices,
// every tiling timed back to back): four waves across K for rows of up to 8
// chunks, eight for longer rows; two rows per workgroup with fp16 x, four with
// fp32 x (more x registers per chunk), eight for int8 weights (half the bytes
// per row). With a fused RMSNorm every workgroup also reads the norm weights,
// so a vocabulary-sized matrix of short rows (the LM head) takes eight rows per
// workgroup: 256000 x 2048 runs in 158.8 us instead of 197.7. Small M keeps
// enough workgroups to fill the GPU.
void pick_tiling(int M, int nch, bool q8, bool x_half, bool norm, int& nr, int& nw) {
    if (nch > 8) {
        nw = 8;
        nr = q8 ? 8 : 4;
    } else {
        nw = nch >= 4 ? 4 : nch >= 2 ? 2 : 1;
        nr = q8 ? 8 : x_half ? 2 : 4;
        if (norm && M >= 65536) nr = 8;
    }
    if (M < 1024) nr = M >= 256 ? (nr < 2 ? nr : 2) : 1;
    nr = mxd::tunable("MV_NR", nr);
    nw = mxd::tunable("MV_NW", nw);
}

template <int WF, typename XT, int NMAT, int OP, int NR, bool RES>
int launch_nwr(const GemvArgs& a, int nw, hipStream_t s) {
    const dim3 grid((a.M + NR - 1) / NR);
    const size_t dyn = dyn_lds(a);
    switch (nw) {
        case 1: hipLaunchKernelGGL((gemv_kernel<WF, XT, NMAT, OP, NR, 1, RES>), grid, dim3(64), dyn, s, a); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<WF, XT, NMAT, OP, NR, 2, RES>), grid, dim3(128), dyn, s, a); break;
        case 4: hipLaunchKernelGGL((gemv_kernel<WF, XT, NMAT, OP, NR, 4, RES>), grid, dim3(256), dyn, s, a); break;
        case 8: hipLaunchKernelGGL((gemv_kernel<WF, XT, NMAT, OP, NR, 8, RES>), grid, dim3(512), dyn, s, a); break;
        default: return mxd::fail(MXD_ERR_INVALID_ARG, "matvec: MV_NW must be 1, 2, 4 or 8 (got %d)", nw);
    }
    return mxd::check_launch("matvec");
}

template <int WF, typename XT, int NMAT, int OP, int NR>
int launch_nw(const GemvArgs& a, int nw, hipStream_t s) {
    if constexpr (res_capable<WF, XT, OP>()) {
        if (a.rsrc) return launch_nwr<WF, XT, NMAT, OP, NR, true>(a, nw, s);
    }
    return launch_nwr<WF, XT, NMAT, OP, NR, false>(a, nw, s);
}

template <int WF, typename XT, int NMAT, int OP>
int launch(const GemvArgs& a, hipStream_t s) {
    constexpr int CH = 64 * WT<WF>::EPL;
    const int nch = (a.K + CH - 1) / CH;
    // MV_ALGO: 0 = row-tiled workgroups, 1 = row streaming (while a row fits
    // 16 waves x 4 chunks), 2 = grid sweep. Defaults from back-to-back sweeps
    // on MI355X: row tiles for rows of up to 8 chunks, row streaming with 16
    // waves for longer rows (4096 x 14336: 6.1 vs 5.8 TB/s fp16, 5.3 vs 4.9
    // TB/s int8).
    //
    // Short fp16 rows (up to 4 chunks, e.g. K = 2048) also stream by rows in
    // two cases, from back-to-back sweeps of the Gemma-2B decode shapes: the
    // gate/up pair (16384 x 2048 x 2 with the fused norm: 22.7 vs 23.8 us, 8
    // waves, 4 workgroups per CU) and small single matrices without a RoPE
    // epilogue (the 2048 x 2048 o projection: 3.95 vs 4.63 us, 4 waves, 8 per
    // CU).
    //
    // A vocabulary-sized matrix of short fp16 rows with the fused norm (the
    // LM head, 256000 x 2048) takes the grid sweep: each wave forms its
    // x * w_norm fragment once for the whole kernel, and each workgroup the
    // rsqrt scale once, instead of once per tile of rows.
    // Back-to-back on MI355X: 157.4 us against 171.7 (row tiles, 8 rows x 4
    // waves) and 161.0 (row streaming).
    const bool short_f16 = WF == MXD_W_F16 && nch <= 4 && OP != EPI_ROPE_KV;
    const bool rows_glu = short_f16 && NMAT == 2;
    const bool rows_small = short_f16 && NMAT == 1 && a.M <= 4096;
    const bool sweep_vocab = short_f16 && NMAT == 1 && a.nw != nullptr && a.M >= 65536;
    // int8 rows of up to 4 chunks against fp16 x (the 14336 x 4096 FFN matrix)
    // stream by rows, 4 waves and 8 workgroups per CU: graph-replayed, three
    // alternating rounds, 12.04-12.07 us against 12.58-12.76 (8-row tiles).
    const bool rows_q8 = WF == MXD_W_Q8B32 && std::is_same<XT, _Float16>::value && NMAT == 1 &&
                         OP != EPI_ROPE_KV && nch <= 4 && a.M >= 8192;
    const bool rows_long = nch > 8 && nch <= RS_MAX_CHUNKS;
    int algo_default = 0;
    if (sweep_vocab)
        algo_default = 2;
    else if (rows_long || rows_glu || rows_small || rows_q8)
        algo_default = 1;
    const int algo = mxd::tunable("MV_ALGO", algo_default);
    if (algo == 1) {
        MXD_REQUIRE(nch <= RS_MAX_CHUNKS, MXD_ERR_UNSUPPORTED, "matvec: row streaming needs K <= %d",
                    RS_MAX_CHUNKS * CH);
        // Long rows: 16 waves, or 14 where 14 waves cover the row's chunks
        // exactly (K = 14336: 28 fp16 chunks as 14 x 2 instead of 16 x 2;
        // 4096 x 14336 fp16 measured 18.9 against 19.3 us). Where neither
        // covers it exactly, 16 (Gemma-4-E2B down, 1536 x 12288: 8.60 against
        // 9.08 us as 14 x 2; 1536 x 6144: 5.52 against 5.62 as 14 x 1).
        const int nw_long = nch % 14 == 0 && nch <= 28 ? 14 : 16;
        // Rows of 3 chunks (K = 1536) keep every wave busy with 4 waves; the
        // gate/up pair then runs 8 workgroups per CU (E2B, 12288 x 1536 x 2
        // with the residual prologue: 15.79 against 18.33 us as 8 waves x 4
        // per CU; 6144 rows: 10.21 against 11.05).
        const bool glu3 = rows_glu && nch <= 3;
        const int nw = mxd::tunable("MV_RS_NW", rows_glu && !glu3 ? 8 : nch <= 4 ? 4 : nch <= 8 ? 8 : nw_long);
        int cpw = (nch + nw - 1) / nw;
        cpw = cpw <= 1 ? 1 : cpw <= 2 ? 2 : 4;
        MXD_REQUIRE(nw * cpw >= nch, MXD_ERR_UNSUPPORTED,
                    "matvec: row streaming with %d waves covers at most %d chunks", nw, nw * 4);
        // The residual prologue is per workgroup (it reads three K-vectors
        // and reduces them before the first row), so a single short-row
        // matrix with it takes 4 workgroups per CU instead of 8 (E2B q|k|v,
        // 2560 x 1536: 5.80 against 6.50 us; q, 2048 x 1536: 5.62 against 6.38).
        const int wg_small = a.rsrc && nw == 4 ? 4 : 32 / nw;
        const int wg_per_cu =
            mxd::tunable("MV_RS_WGCU", glu3 ? 8 : rows_glu ? 4 : nw >= 16 ? 2 : wg_small);
        return launch_rows<WF, XT, NMAT, OP>(a, nw, cpw, wg_per_cu, s);
    }
    if (algo == 2) {
        MXD_REQUIRE(nch <= RS_MAX_CHUNKS, MXD_ERR_UNSUPPORTED, "matvec: sweep needs K <= %d", RS_MAX_CHUNKS * CH);
        const int nw = mxd::tunable("MV_SW_NW", nch <= 4 ? 4 : nch <= 8 ? 8 : 16);
        int cpw = (nch + nw - 1) / nw;
        cpw = cpw <= 1 ? 1 : cpw <= 2 ? 2 : 4;
        MXD_REQUIRE(nw * cpw >= nch, MXD_ERR_UNSUPPORTED, "matvec: sweep with %d waves covers at most %d chunks",
                    nw, nw * 4);
        const int wg_per_cu = mxd::tunable("MV_SW_WGCU", 32 / nw > 0 ? 32 / nw : 1);
        return launch_sweep<WF, XT, NMAT, OP>(a, nw, cpw, wg_per_cu, s);
    }
    int nr, nw;
    pick_tiling(a.M, nch, WF == MXD_W_Q8B32, sizeof(XT) == 2, a.nw != nullptr, nr, nw);
    switch (nr) {
        case 1: return launch_nw<WF, XT, NMAT, OP, 1>(a, nw, s);
        case 2: return launch_nw<WF, XT, NMAT, OP, 2>(a, nw, s);
        case 4: return launch_nw<WF, XT, NMAT, OP, 4>(a, nw, s);
        case 8: return launch_nw<WF, XT, NMAT, OP, 8>(a, nw, s);
        default: return mxd::fail(MXD_ERR_INVALID_ARG, "matvec: MV_NR must be 1, 2, 4 or 8 (got %d)", nr);
    }
}

template <int WF, typename XT>
int launch_epi(const GemvArgs& a, int epi, hipStream_t s) {
    switch (epi) {
        case MXD_EPI_STORE: return launch<WF, XT, 1, MXD_EPI_STORE>(a, s);
        case MXD_EPI_ADD: return launch<WF, XT, 1, MXD_EPI_ADD>(a, s);
        case MXD_EPI_GELU_MUL: return launch<WF, XT, 1, MXD_EPI_GELU_MUL>(a, s);
        default: return mxd::fail(MXD_ERR_INVALID_ARG, "matvec: unknown epilogue %d", epi);
    }
}

template <int WF, typename XT>
int launch_act(const GemvArgs& a, int act, hipStream_t s) {
    switch (act) {
        case MXD_ACT_GELU_TANH: return launch<WF, XT, 2, MXD_ACT_GELU_TANH>(a, s);
        case MXD_ACT_SILU: return launch<WF, XT, 2, MXD_ACT_SILU>(a, s);
        default: return mxd::fail(MXD_ERR_INVALID_ARG, "matvec_gate_up: unknown activation %d", act);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_common(const char* fn, const void* W, const void* x, const float* y, int M, int K) {
    MXD_REQUIRE(W && x && y, MXD_ERR_INVALID_ARG, "%s: null pointer", fn);
    MXD_REQUIRE(M > 0 && K > 0, MXD_ERR_INVALID_ARG, "%s: M=%d K=%d must be positive", fn, M, K);
    MXD_REQUIRE(aligned16(W) && aligned16(x), MXD_ERR_UNSUPPORTED, "%s: W and x must be 16-byte aligned", fn);
    return MXD_OK;
}

}  // namespace

extern "C" int mxd_gemv_f32(const float* W, const float* x, float* y, int M, int K, mxd_stream_t stream) {
    if (int rc = check_common("mxd_gemv_f32", W, x, y, M, K)) return rc;
    MXD_REQUIRE(K % 4 == 0, MXD_ERR_UNSUPPORTED, "mxd_gemv_f32: K=%d must be a multiple of 4", K);
    GemvArgs a{{W, nullptr}, {nullptr, nullptr}, x, y, nullptr, M, K};
    return launch<WF_F32, float, 1, MXD_EPI_STORE>(a, mxd::as_stream(stream));
}

extern "C" int mxd_matvec_f16(const uint16_t* W, const void* x, int x_dtype, float* y, int M, int K, int epilogue,
                              const float* aux, mxd_stream_t stream) {
    if (int rc = check_common("mxd_matvec_f16", W, x, y, M, K)) return rc;
    MXD_REQUIRE(K % 8 == 0, MXD_ERR_UNSUPPORTED, "mxd_matvec_f16: K=%d must be a multiple of 8", K);
    MXD_REQUIRE(epilogue != MXD_EPI_GELU_MUL || aux, MXD_ERR_INVALID_ARG, "mxd_matvec_f16: GELU_MUL needs aux");
    GemvArgs a{{W, nullptr}, {nullptr, nullptr}, x, y, aux, M, K};
    hipStream_t s = mxd::as_stream(stream);
    if (x_dtype == MXD_F32) return launch_epi<MXD_W_F16, float>(a, epilogue, s);
    if (x_dtype == MXD_F16) return launch_epi<MXD_W_F16, _Float16>(a, epilogue, s);
    return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_matvec_f16: x_dtype %d", x_dtype);
}

namespace mxd {

// fp16 or int8 matvec with fp32 x rounded to fp16 as it is loaded (the
// per-row path of the batched products with fp32 activations).
int matvec_xr16(int w_format, const void* W, const uint16_t* scales, const float* x, float* y, int M, int K,
                int epilogue, hipStream_t s) {
    if (int rc = check_common("matvec (fp32 x rounded to fp16)", W, x, y, M, K)) return rc;
    GemvArgs a{{W, nullptr}, {scales, nullptr}, x, y, nullptr, M, K};
    a.xr16 = 1;
    if (w_format == MXD_W_Q8B32) return launch_epi<MXD_W_Q8B32, float>(a, epilogue, s);
    return launch_epi<MXD_W_F16, float>(a, epilogue, s);
}

}  // namespace mxd

extern "C" int mxd_matvec_q8b32(const int8_t* Wq, const uint16_t* scales, const void* x, int x_dtype, float* y, int M,
                                int K, int epilogue, const float* aux, mxd_stream_t stream) {
    if (int rc = check_common("mxd_matvec_q8b32", Wq, x, y, M, K)) return rc;
    MXD_REQUIRE(scales, MXD_ERR_INVALID_ARG, "mxd_matvec_q8b32: null scales");
    MXD_REQUIRE(K % 32 == 0, MXD_ERR_UNSUPPORTED, "mxd_matvec_q8b32: K=%d must be a multiple of 32", K);
    MXD_REQUIRE(epilogue != MXD_EPI_GELU_MUL || aux, MXD_ERR_INVALID_ARG, "mxd_matvec_q8b32: GELU_MUL needs aux");
    GemvArgs a{{Wq, nullptr}, {scales, nullptr}, x, y, aux, M, K};
    hipStream_t s = mxd::as_stream(stream);
    if (x_dtype == MXD_F32) return launch_epi<MXD_W_Q8B32, float>(a, epilogue, s);
    if (x_dtype == MXD_F16) return launch_epi<MXD_W_Q8B32, _Float16>(a, epilogue, s);
    return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_matvec_q8b32: x_dtype %d", x_dtype);
}

extern "C" int mxd_matvec_gate_up(int w_format, const void* Wg, const uint16_t* sg, const void* Wu,
                                  const uint16_t* su, const void* x, int x_dtype, float* h, int F, int K, int act,
                                  mxd_stream_t stream) {
    if (int rc = check_common("mxd_matvec_gate_up", Wg, x, h, F, K)) return rc;
    MXD_REQUIRE(Wu && aligned16(Wu), MXD_ERR_INVALID_ARG, "mxd_matvec_gate_up: Wu null or not 16-byte aligned");
    GemvArgs a{{Wg, Wu}, {sg, su}, x, h, nullptr, F, K};
    hipStream_t s = mxd::as_stream(stream);
    if (w_format == MXD_W_F16) {
        MXD_REQUIRE(K % 8 == 0, MXD_ERR_UNSUPPORTED, "mxd_matvec_gate_up: K=%d must be a multiple of 8", K);
        if (x_dtype == MXD_F32) return launch_act<MXD_W_F16, float>(a, act, s);
        if (x_dtype == MXD_F16) return launch_act<MXD_W_F16, _Float16>(a, act, s);
    } else if (w_format == MXD_W_Q8B32) {
        MXD_REQUIRE(sg && su, MXD_ERR_INVALID_ARG, "mxd_matvec_gate_up: int8 weights need scales");
        MXD_REQUIRE(K % 32 == 0, MXD_ERR_UNSUPPORTED, "mxd_matvec_gate_up: K=%d must be a multiple of 32", K);
        if (x_dtype == MXD_F32) return launch_act<MXD_W_Q8B32, float>(a, act, s);
        if (x_dtype == MXD_F16) return launch_act<MXD_W_Q8B32, _Float16>(a, act, s);
    } else {
        return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_matvec_gate_up: weight format %d", w_format);
    }
    return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_matvec_gate_up: x_dtype %d", x_dtype);
}

// ---------------------------------------------------------------------------
// Fused decode-step operators: RMSNorm folded into the matvec's x loads, and
// the q|k|v projection with RoPE + KV append in its epilogue. Each removes a
// launch (and an activation round trip) per layer from the decode step.
// ---------------------------------------------------------------------------

namespace {

int check_norm(const char* fn, const void* W, const float* x, const float* nw, const float* y, int M, int K) {
    if (int rc = check_common(fn, W, x, y, M, K)) return rc;
    MXD_REQUIRE(nw && aligned16(nw), MXD_ERR_INVALID_ARG, "%s: norm weight null or not 16-byte aligned", fn);
    MXD_REQUIRE(K % 8 == 0, MXD_ERR_UNSUPPORTED, "%s: K=%d must be a multiple of 8", fn, K);
    return MXD_OK;
}

}  // namespace

extern "C" int mxd_matvec_f16_rmsnorm(const uint16_t* W, const float* x, const float* norm_w, float eps, int plus_one,
                                      float* y, int M, int K, int epilogue, const float* aux, mxd_stream_t stream) {
    if (int rc = check_norm("mxd_matvec_f16_rmsnorm", W, x, norm_w, y, M, K)) return rc;
    MXD_REQUIRE(epilogue != MXD_EPI_GELU_MUL || aux, MXD_ERR_INVALID_ARG, "mxd_matvec_f16_rmsnorm: GELU_MUL needs aux");
    GemvArgs a{{W, nullptr}, {nullptr, nullptr}, x, y, aux, M, K};
    a.nw = norm_w;
    a.eps = eps;
    a.plus_one = plus_one;
    return launch_epi<MXD_W_F16, float>(a, epilogue, mxd::as_stream(stream));
}

extern "C" int mxd_gate_up_rmsnorm(const uint16_t* Wg, const uint16_t* Wu, const float* x, const float* norm_w,
                                   float eps, int plus_one, float* h, int F, int K, int act, mxd_stream_t stream) {
    if (int rc = check_norm("mxd_gate_up_rmsnorm", Wg, x, norm_w, h, F, K)) return rc;
    MXD_REQUIRE(Wu && aligned16(Wu), MXD_ERR_INVALID_ARG, "mxd_gate_up_rmsnorm: Wu null or not 16-byte aligned");
    GemvArgs a{{Wg, Wu}, {nullptr, nullptr}, x, h, nullptr, F, K};
    a.nw = norm_w;
    a.eps = eps;
    a.plus_one = plus_one;
    return launch_act<MXD_W_F16, float>(a, act, mxd::as_stream(stream));
}

namespace {

int check_residual(const char* fn, const float* x, const float* res_src, const float* res_w, const float* x_out) {
    MXD_REQUIRE(res_src && res_w && x_out, MXD_ERR_INVALID_ARG, "%s: null residual pointer", fn);
    MXD_REQUIRE(x_out != x && x_out != res_src, MXD_ERR_INVALID_ARG, "%s: x_out must not alias x or res_src", fn);
    MXD_REQUIRE(aligned16(res_src) && aligned16(res_w) && aligned16(x_out), MXD_ERR_UNSUPPORTED,
                "%s: residual pointers must be 16-byte aligned", fn);
    return MXD_OK;
}

}  // namespace

extern "C" int mxd_matvec_f16_residual(const uint16_t* W, const float* x, const float* res_src, const float* res_w,
                                       float res_post, float* x_out, const float* norm_w, float eps, int plus_one,
                                       float* y, int M, int K, int epilogue, const float* aux, mxd_stream_t stream) {
    const char* fn = "mxd_matvec_f16_residual";
    if (norm_w) {
        if (int rc = check_norm(fn, W, x, norm_w, y, M, K)) return rc;
    } else {
        if (int rc = check_common(fn, W, x, y, M, K)) return rc;
        MXD_REQUIRE(K % 8 == 0, MXD_ERR_UNSUPPORTED, "%s: K=%d must be a multiple of 8", fn, K);
    }
    if (int rc = check_residual(fn, x, res_src, res_w, x_out)) return rc;
    MXD_REQUIRE(epilogue != MXD_EPI_GELU_MUL || aux, MXD_ERR_INVALID_ARG, "%s: GELU_MUL needs aux", fn);
    GemvArgs a{{W, nullptr}, {nullptr, nullptr}, x, y, aux, M, K};
    a.nw = norm_w;
    a.eps = eps;
    a.plus_one = plus_one;
    a.rsrc = res_src;
    a.rw = res_w;
    a.rpost = res_post;
    a.rout = x_out;
    return launch_epi<MXD_W_F16, float>(a, epilogue, mxd::as_stream(stream));
}

extern "C" int mxd_gate_up_residual(const uint16_t* Wg, const uint16_t* Wu, const float* x, const float* res_src,
                                    const float* res_w, float res_post, float* x_out, const float* norm_w, float eps,
                                    int plus_one, float* h, int F, int K, int act, mxd_stream_t stream) {
    const char* fn = "mxd_gate_up_residual";
    if (int rc = check_norm(fn, Wg, x, norm_w, h, F, K)) return rc;
    MXD_REQUIRE(Wu && aligned16(Wu), MXD_ERR_INVALID_ARG, "%s: Wu null or not 16-byte aligned", fn);
    if (int rc = check_residual(fn, x, res_src, res_w, x_out)) return rc;
    GemvArgs a{{Wg, Wu}, {nullptr, nullptr}, x, h, nullptr, F, K};
    a.nw = norm_w;
    a.eps = eps;
    a.plus_one = plus_one;
    a.rsrc = res_src;
    a.rw = res_w;
    a.rpost = res_post;
    a.rout = x_out;
    return launch_act<MXD_W_F16, float>(a, act, mxd::as_stream(stream));
}

extern "C" int mxd_qkv_rope_kv(const uint16_t* Wqkv, const float* x, const float* norm_w, float eps, int plus_one,
                               float* q, uint16_t* kcache, uint16_t* vcache, const float* inv_freq, int n_heads,
                               int n_kv_heads, int head_dim, int K, int max_ctx, int pos, const int32_t* pos_dev,
                               mxd_stream_t stream) {
    const int M = (n_heads + 2 * n_kv_heads) * head_dim;
    MXD_REQUIRE(n_heads > 0 && n_kv_heads > 0, MXD_ERR_INVALID_ARG, "mxd_qkv_rope_kv: head counts");
    MXD_REQUIRE(head_dim > 0 && head_dim % 32 == 0, MXD_ERR_UNSUPPORTED, "mxd_qkv_rope_kv: head_dim=%d", head_dim);
    MXD_REQUIRE(max_ctx > 0 && max_ctx % 32 == 0, MXD_ERR_UNSUPPORTED, "mxd_qkv_rope_kv: max_ctx=%d", max_ctx);
    MXD_REQUIRE(pos_dev || (pos >= 0 && pos < max_ctx), MXD_ERR_INVALID_ARG, "mxd_qkv_rope_kv: pos %d outside [0, %d)",
                pos, max_ctx);
    MXD_REQUIRE(kcache && vcache && inv_freq, MXD_ERR_INVALID_ARG, "mxd_qkv_rope_kv: null cache or inv_freq");
    if (norm_w) {
        if (int rc = check_norm("mxd_qkv_rope_kv", Wqkv, x, norm_w, q, M, K)) return rc;
    } else {
        if (int rc = check_common("mxd_qkv_rope_kv", Wqkv, x, q, M, K)) return rc;
        MXD_REQUIRE(K % 8 == 0, MXD_ERR_UNSUPPORTED, "mxd_qkv_rope_kv: K=%d must be a multiple of 8", K);
    }
    GemvArgs a{{Wqkv, nullptr}, {nullptr, nullptr}, x, q, nullptr, M, K};
    a.nw = norm_w;
    a.eps = eps;
    a.plus_one = plus_one;
    a.inv_freq = inv_freq;
    a.kcache = kcache;
    a.vcache = vcache;
    a.pos_dev = pos_dev;
    a.pos = pos;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.hd = head_dim;
    a.max_ctx = max_ctx;
    int nr, nw;
    pick_tiling(M, (K + 511) / 512, false, false, false, nr, nw);
    nr = nr < 2 ? 2 : (nr & ~1);  // rotation pairs stay inside one workgroup
    hipStream_t s = mxd::as_stream(stream);
    switch (nr) {
        case 2: return launch_nw<MXD_W_F16, float, 1, EPI_ROPE_KV, 2>(a, nw, s);
        case 4: return launch_nw<MXD_W_F16, float, 1, EPI_ROPE_KV, 4>(a, nw, s);
        default: return launch_nw<MXD_W_F16, float, 1, EPI_ROPE_KV, 8>(a, nw, s);
    }
}

extern "C" int mxd_matvec_f16_attn_merge(const uint16_t* W, const float* partials, int n_splits, int n_heads,
                                         int head_dim, int max_ctx, int n_keys, const int32_t* pos_dev, float* y,
                                         int M, int epilogue, const float* aux, mxd_stream_t stream) {
    return mxd_matvec_f16_attn_merge_window(W, partials, n_splits, n_heads, head_dim, max_ctx, n_keys, pos_dev, 0, y,
                                            M, epilogue, aux, stream);
}

extern "C" int mxd_matvec_f16_attn_merge_window(const uint16_t* W, const float* partials, int n_splits, int n_heads,
                                                int head_dim, int max_ctx, int n_keys, const int32_t* pos_dev,
                                                int window, float* y, int M, int epilogue, const float* aux,
                                                mxd_stream_t stream) {
    const int K = n_heads * head_dim;
    MXD_REQUIRE(window >= 0, MXD_ERR_INVALID_ARG, "mxd_matvec_f16_attn_merge: window=%d", window);
    if (int rc = check_common("mxd_matvec_f16_attn_merge", W, partials, y, M, K)) return rc;
    MXD_REQUIRE(n_splits >= 1 && n_splits <= MERGE_MAX_SPLITS, MXD_ERR_UNSUPPORTED,
                "mxd_matvec_f16_attn_merge: n_splits=%d outside [1, %d]", n_splits, MERGE_MAX_SPLITS);
    MXD_REQUIRE(head_dim > 0 && head_dim % 8 == 0, MXD_ERR_UNSUPPORTED,
                "mxd_matvec_f16_attn_merge: head_dim=%d must be a multiple of 8", head_dim);
    MXD_REQUIRE(max_ctx > 0, MXD_ERR_INVALID_ARG, "mxd_matvec_f16_attn_merge: max_ctx=%d", max_ctx);
    MXD_REQUIRE(pos_dev || (n_keys >= 0 && n_keys <= max_ctx), MXD_ERR_INVALID_ARG,
                "mxd_matvec_f16_attn_merge: n_keys=%d outside [0, max_ctx=%d]", n_keys, max_ctx);
    MXD_REQUIRE(epilogue != MXD_EPI_GELU_MUL || aux, MXD_ERR_INVALID_ARG,
                "mxd_matvec_f16_attn_merge: GELU_MUL needs aux");
    GemvArgs a{{W, nullptr}, {nullptr, nullptr}, partials, y, aux, M, K};
    a.mpo = partials;
    a.mpml = partials + (size_t)n_splits * K;
    a.msplits = n_splits;
    a.n_heads = n_heads;
    a.hd = head_dim;
    a.max_ctx = max_ctx;
    a.n_keys = n_keys;
    a.pos_dev = pos_dev;
    a.mwindow = window;
    // Row tiles (every workgroup merges the x it reads, so fewer, taller
    // tiles read fewer partials): 8 rows from 2048 rows on, 4 from 1024
    // (Gemma-4-E2B, 1536 rows: decode 519 -> 538 tok/s against 2-row tiles;
    // 8-row tiles, 192 workgroups, 534).
    int nr, nw;
    pick_tiling(M, (K + 511) / 512, false, false, false, nr, nw);
    hipStream_t s = mxd::as_stream(stream);
    auto go = [&](auto nrc) -> int {
        constexpr int NR = decltype(nrc)::value;
        switch (epilogue) {
            case MXD_EPI_STORE: return launch_nw<MXD_W_F16, float, 1, MXD_EPI_STORE, NR>(a, nw, s);
            case MXD_EPI_ADD: return launch_nw<MXD_W_F16, float, 1, MXD_EPI_ADD, NR>(a, nw, s);
            case MXD_EPI_GELU_MUL: return launch_nw<MXD_W_F16, float, 1, MXD_EPI_GELU_MUL, NR>(a, nw, s);
            default: return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_matvec_f16_attn_merge: unknown epilogue %d", epilogue);
        }
    };
    const int nrm = mxd::tunable("MV_MERGE_NR", M >= 2048 ? 8 : M >= 1024 ? 4 : M >= 256 ? 2 : 1);
    if (nrm >= 8) return go(std::integral_constant<int, 8>{});
    if (nrm >= 4) return go(std::integral_constant<int, 4>{});
    if (nrm >= 2) return go(std::integral_constant<int, 2>{});
    return go(std::integral_constant<int, 1>{});
}
