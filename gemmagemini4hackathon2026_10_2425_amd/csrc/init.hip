// Synthetic weights: a counter-based normal generator whose every bit the
// oracle reproduces on the CPU.
//
// Element i of tensor (seed, tensor_id):
//   key = mix(mix(seed) ^ tensor_id)
//   h0 = mix(key + 2i), h1 = mix(key + 2i + 1)     (mix = splitmix64 output)
//   c  = sum of the eight 16-bit fields of h0, h1  - 4 * 65535
//   v  = float(c) * k,  k = float(stddev / sqrt(8 * (65536^2 - 1) / 12))
// c is an integer below 2^19, so float(c) is exact and v is one correctly
// rounded fp32 multiply on any IEEE machine; fp16 output rounds to nearest even.
#include "internal.hpp"

#include <math.h>

namespace {

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ int32_t sum16x4(uint64_t h) {
    return (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) + (int32_t)((h >> 32) & 0xFFFF) +
           (int32_t)(h >> 48);
}

// SHIFT: fp32 v + shift (the Gemma-4 norm weights, 1 + N(0, s^2)).
template <int DT, bool SHIFT = false>
__global__ void __launch_bounds__(256) fill_normal_kernel(void* dst, uint64_t n, uint64_t key, float k,
                                                          float shift = 0.0f) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t h0 = mix64(key + 2 * i);
        const uint64_t h1 = mix64(key + 2 * i + 1);
        const int32_t c = sum16x4(h0) + sum16x4(h1) - 4 * 65535;
        float v = (float)c * k;
        // Keep the fp32 product: without this the compiler folds the multiply
        // and the fp16 conversion into one mixed-precision FMA that rounds once,
        // straight to fp16, which is not the value this generator defines.
        asm volatile("" : "+v"(v));
        if (SHIFT) v += shift;
        if (DT == MXD_F32)
            static_cast<float*>(dst)[i] = v;
        else
            static_cast<uint16_t*>(dst)[i] = mxd::f2h_bits(v);
    }
}

}  // namespace

int mxd::fill_normal_dev(void* dst, int dtype, uint64_t n, uint64_t seed, uint64_t tensor_id, float stddev,
                         float shift, hipStream_t s) {
    MXD_REQUIRE(dtype == MXD_F32 || dtype == MXD_F16, MXD_ERR_INVALID_ARG, "mxd_fill_normal: dtype %d", dtype);
    MXD_REQUIRE(shift == 0.0f || dtype == MXD_F32, MXD_ERR_INVALID_ARG, "mxd_fill_normal: shift needs fp32");
    if (n == 0) return MXD_OK;
    MXD_REQUIRE(dst != nullptr, MXD_ERR_INVALID_ARG, "mxd_fill_normal: null dst");
    const uint64_t key = mix64(mix64(seed) ^ tensor_id);
    const float k = (float)((double)stddev / sqrt(8.0 * (65536.0 * 65536.0 - 1.0) / 12.0));
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    const dim3 grid((unsigned)blocks), block(256);
    if (shift != 0.0f)
        hipLaunchKernelGGL((fill_normal_kernel<MXD_F32, true>), grid, block, 0, s, dst, n, key, k, shift);
    else if (dtype == MXD_F32)
        hipLaunchKernelGGL(fill_normal_kernel<MXD_F32>, grid, block, 0, s, dst, n, key, k, 0.0f);
    else
        hipLaunchKernelGGL(fill_normal_kernel<MXD_F16>, grid, block, 0, s, dst, n, key, k, 0.0f);
    return mxd::check_launch("mxd_fill_normal");
}

extern "C" int mxd_fill_normal(void* dst, int dtype, uint64_t n, uint64_t seed, uint64_t tensor_id,
                               float stddev, mxd_stream_t stream) {
    return mxd::fill_normal_dev(dst, dtype, n, seed, tensor_id, stddev, 0.0f, mxd::as_stream(stream));
}
