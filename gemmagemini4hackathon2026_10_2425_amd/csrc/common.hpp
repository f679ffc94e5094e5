// Shared device helpers and host-side error plumbing for libmxdecode.
//
// Everything here is written for gfx950 (CDNA4): 64-lane wavefronts, DPP row
// operations for the first reduction steps, ds_bpermute for the cross-row ones.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/mxdecode.h"

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Host-side error state (thread-local), shared by every entry point.
// ---------------------------------------------------------------------------
namespace mxd {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps the last launch status to an MXD code, recording the HIP message.
int check_launch(const char* what);

inline hipStream_t as_stream(mxd_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Tunables (mirrors the reference's `--define NAME=VALUE` kernel knobs).
int tunable(const char* name, int fallback);

}  // namespace mxd

#define MXD_REQUIRE(cond, code, ...)                 \
    do {                                             \
        if (!(cond)) return mxd::fail((code), __VA_ARGS__); \
    } while (0)

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
namespace mxd {

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
// Steps: swap pairs, swap pair-of-pairs (quad_perm), rotate 4 and 8 inside
// each 16-lane row (DPP), then combine the four rows with bpermute.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x124>(v));
    v = fmaxf(v, dpp_f32<0x128>(v));
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

__device__ __forceinline__ float h2f(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ uint16_t f2h_bits(float f) {
    _Float16 h = (_Float16)f;  // round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ h2_t as_h2(uint32_t u) {
    h2_t h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

// Four signed int8 values packed in a dword -> two half2 holding the exact
// integers. q ^ 0x80 is the unsigned byte q + 128; 0x6400 | b is the fp16
// value 1024 + b, so subtracting 1152 leaves q exactly.
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, h2_t& lo, h2_t& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x07010700u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x07030702u);
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = as_h2(a) - bias;
    hi = as_h2(b) - bias;
}

__device__ __forceinline__ float gelu_tanh(float x) {
    // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), accurate tanh.
    return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Offsets (in halfs) of position k (0..31) and dim d inside a 32-position KV
// cache tile, in the MFMA operand order the attention kernel loads (layouts
// spelled out in include/mxdecode.h). The tile of position p of kv head h
// starts at (h * max_ctx + (p & ~31)) * hd.
__device__ __forceinline__ int k_tile_offset(int k, int d, int hd) {
    const int t = (k >> 2) & 1, col = ((k >> 3) << 2) | (k & 3);
    const int c = d >> 5, g = (d >> 3) & 3, e = d & 7;
    return ((t * (hd >> 5) + c) * 64 + g * 16 + col) * 8 + e;
}

__device__ __forceinline__ int v_tile_offset(int k, int d) {
    const int dt = d >> 4, col = d & 15, g = k >> 3, j = k & 7;
    return (dt * 64 + g * 16 + col) * 8 + j;
}

// Paged KV cache: a page holds PAGE_KEYS positions of every kv head; the
// (page, kv head) slab of PAGE_KEYS * hd fp16 values starts at
// (page * n_kv + kvh) * PAGE_KEYS * hd. A slab is one half of a 32-position
// tile of the contiguous layout above, with that half's pieces made
// contiguous, so a 32-key block is two pages and every MFMA operand is two
// 512-byte runs. Offsets (in halfs) of key r (0..15) and dim d in a slab:
//   K: ((((d >> 5) * 2 + ((r >> 2) & 1)) * 4 + ((d >> 3) & 3)) * 8 + rr) * 8 + (d & 7),
//      rr = ((r >> 3) << 2) | (r & 3)
//   V: (((d >> 4) * 2 + (r >> 3)) * 16 + (d & 15)) * 8 + (r & 7)
constexpr int PAGE_KEYS = 16;

__host__ __device__ __forceinline__ int k_page_offset(int r, int d) {
    const int rr = ((r >> 3) << 2) | (r & 3);
    return ((((d >> 5) * 2 + ((r >> 2) & 1)) * 4 + ((d >> 3) & 3)) * 8 + rr) * 8 + (d & 7);
}

__host__ __device__ __forceinline__ int v_page_offset(int r, int d) {
    return (((d >> 4) * 2 + (r >> 3)) * 16 + (d & 15)) * 8 + (r & 7);
}


// ---------------------------------------------------------------------------
// Tagged handoff words. A kernel whose workgroups pass values to each other
// (the fused decode attention block) stores each fp32 value with a 32-bit tag
// in one 8-byte word, written and read whole with agent-scope relaxed atomics
// (coherent across the XCDs' L2s without fences). A reader takes a word only
// once it carries the current launch's tag; stale words from earlier launches
// carry older tags. Waits are bounded: past TAG_SPIN_LIMIT polls the reader
// records an error in *err and goes on with what it read, and once the error
// is set every later wait returns at once.
// ---------------------------------------------------------------------------
constexpr unsigned TAG_SPIN_LIMIT = 1u << 16;

__device__ __forceinline__ void tag_put(uint64_t* p, uint32_t tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t tag_peek(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool tag_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

__device__ __forceinline__ float tag_value(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Loads N words per lane (p[i], or nothing where p[i] is null) until every
// lane of the wave holds words carrying `tag`; returns their values.
template <int N>
__device__ __forceinline__ void tag_wait(const uint64_t* const (&p)[N], uint32_t tag, float (&v)[N], int* err) {
    unsigned spins = 0;
    const bool failed = err && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    while (true) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (!p[i]) continue;
            const uint64_t w = tag_peek(p[i]);
            ok = ok && tag_ok(w, tag);
            v[i] = tag_value(w);
        }
        if (__all(ok) || failed) return;
        if (++spins > TAG_SPIN_LIMIT) {
            if (err) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

}  // namespace mxd
