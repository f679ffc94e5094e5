// Greedy sampling: tokens[out_idx] = argmax(logits), ties to the lowest index
// (KL/kernels.metal:310-345). As in the reference's `v > best` scan from
// best = -inf, NaN and -inf logits are never selected, and a row with nothing
// else gives token 0.
//
// Many workgroups scan the logits; each folds (value, index) into one 64-bit
// key, key = orderable(value) << 32 | ~index, so a larger key is a larger
// value and, for equal values, a smaller index. One atomicMax per workgroup
// combines them, and the last workgroup to finish (ticket counter) writes the
// token and clears both words, leaving the workspace zeroed for the next call
// without a memset (safe inside a captured graph).
#include "internal.hpp"

namespace {

constexpr int AM_THREADS = 256;
constexpr int AM_PER_THREAD = 16;

struct ArgmaxWs {
    unsigned long long best;
    unsigned int ticket;
    unsigned int pad;
};

// Key 0 (never selected) for NaN and -inf; otherwise the value's bits mapped
// to an unsigned order above 0, then the inverted index.
__device__ __forceinline__ unsigned long long pack(float v, int idx) {
    if (!(v > -INFINITY)) return 0ull;
    uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);  // -0 ties with +0
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)(~(uint32_t)idx);
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

__device__ __forceinline__ unsigned long long shfl_xor64(unsigned long long v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((unsigned long long)hi << 32) | lo;
}

__global__ void __launch_bounds__(AM_THREADS)
argmax_kernel(const float* __restrict__ logits, int32_t* __restrict__ tokens, int N, int out_idx, int32_t* pos_dev,
              int advance, ArgmaxWs* ws, int32_t* host_tokens) {
    __shared__ unsigned long long wbest[AM_THREADS / 64];
    __shared__ bool last;
    unsigned long long best = 0;  // below every real key
    const int stride = gridDim.x * AM_THREADS;
    // The grid covers N with AM_PER_THREAD values per thread (up to 1024
    // workgroups): a thread's loads all go out before the first compare
    // (256000 logits on MI355X: 5.24 against 6.63 us as a loop of loads).
    int i = blockIdx.x * AM_THREADS + threadIdx.x;
    float v[AM_PER_THREAD];
#pragma unroll
    for (int k = 0; k < AM_PER_THREAD; ++k) {
        const int j = i + k * stride;
        v[k] = j < N ? logits[j] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < AM_PER_THREAD; ++k) best = umax64(best, pack(v[k], i + k * stride));
    for (i += AM_PER_THREAD * stride; i < N; i += stride) best = umax64(best, pack(logits[i], i));
    for (int m = 1; m < 64; m <<= 1) best = umax64(best, shfl_xor64(best, m));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = wbest[0];
        for (int w = 1; w < AM_THREADS / 64; ++w) b = umax64(b, wbest[w]);
        atomicMax(&ws->best, b);
        __threadfence();
        last = atomicAdd(&ws->ticket, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (last && threadIdx.x == 0) {
        __threadfence();
        const unsigned long long b = atomicMax(&ws->best, 0ull);
        // With pos_dev (a replayed decode step) the token goes to tokens[pos + 1]
        // and, with advance, the step position moves on by one.
        if (pos_dev) out_idx = pos_dev[0] + 1;
        const int32_t tok = b == 0ull ? 0 : (int32_t)(~(uint32_t)(b & 0xFFFFFFFFull));
        tokens[out_idx] = tok;
        if (host_tokens) host_tokens[out_idx] = tok;
        if (pos_dev && advance) pos_dev[0] = out_idx;
        atomicExch(&ws->best, 0ull);
        atomicExch(&ws->ticket, 0u);
    }
}

}  // namespace

extern "C" size_t mxd_argmax_workspace_size(int N) {
    (void)N;
    return sizeof(ArgmaxWs);
}

extern "C" int mxd_argmax(const float* logits, int32_t* tokens, int N, int out_idx, void* workspace, size_t ws_bytes,
                          mxd_stream_t stream) {
    MXD_REQUIRE(logits && tokens, MXD_ERR_INVALID_ARG, "mxd_argmax: null pointer");
    MXD_REQUIRE(N > 0 && out_idx >= 0, MXD_ERR_INVALID_ARG, "mxd_argmax: N=%d out_idx=%d", N, out_idx);
    MXD_REQUIRE(workspace && ws_bytes >= sizeof(ArgmaxWs), MXD_ERR_WORKSPACE,
                "mxd_argmax: workspace of %zu bytes needed", sizeof(ArgmaxWs));
    MXD_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 7) == 0, MXD_ERR_UNSUPPORTED,
                "mxd_argmax: workspace must be 8-byte aligned");
    return mxd::argmax_dev(logits, tokens, N, out_idx, nullptr, false, workspace, mxd::as_stream(stream));
}

namespace mxd {

int argmax_dev(const float* logits, int32_t* tokens, int N, int out_idx, int32_t* pos_dev, bool advance,
               void* workspace, hipStream_t s, int32_t* host_tokens) {
    int blocks = (N + AM_THREADS * AM_PER_THREAD - 1) / (AM_THREADS * AM_PER_THREAD);
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(AM_THREADS), 0, s, logits, tokens, N, out_idx, pos_dev,
                       advance ? 1 : 0, static_cast<ArgmaxWs*>(workspace), host_tokens);
    return check_launch("argmax");
}

}  // namespace mxd
