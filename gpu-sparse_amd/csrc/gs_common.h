// Internal helpers shared by the gfx950 kernels of libgpusparse.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>
#include <stdio.h>

#include "gpusparse.h"

// ------------------------------------------------------------------ errors

void gs_set_error(const char *fmt, ...);

#define GS_CHECK_HIP(expr)                                                               \
    do {                                                                                 \
        hipError_t _e = (expr);                                                          \
        if (_e != hipSuccess) {                                                          \
            gs_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                         __LINE__);                                                      \
            return GS_EHIP;                                                              \
        }                                                                                \
    } while (0)

#define GS_CHECK_LAUNCH() GS_CHECK_HIP(hipGetLastError())

#define GS_REQUIRE(cond, ...)         \
    do {                              \
        if (!(cond)) {                \
            gs_set_error(__VA_ARGS__); \
            return GS_EINVAL;         \
        }                             \
    } while (0)

static inline hipStream_t gs_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

static inline unsigned gs_blocks(int64_t n, int per_block, int64_t cap = 1 << 20) {
    int64_t b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

// 256-byte aligned bump allocator over a caller workspace.
struct gs_arena {
    char *base;
    size_t used;
    size_t cap;
    template <class T>
    T *take(size_t n) {
        size_t off = (used + 255) & ~size_t(255);
        used = off + n * sizeof(T);
        return reinterpret_cast<T *>(base ? base + off : nullptr);
    }
    bool ok() const { return used <= cap; }
};

// ------------------------------------------------------------------ device helpers

constexpr int GS_WAVE = 64;
constexpr int kHeavyTerms = GS_HEAVY_TERMS;  // most frequent terms: the hybrid search's matrix-product terms
constexpr int kSignTerms = 64;               // the first of them sign a query for grouping (a 64-bit mask)
static_assert(kHeavyTerms == 64 || kHeavyTerms == 128 || kHeavyTerms == 256, "heavy terms: 64, 128 or 256");

__device__ __forceinline__ int gs_lane() { return (int)(threadIdx.x & (GS_WAVE - 1)); }

__device__ __forceinline__ uint64_t gs_lanemask_lt() {
    return (1ull << gs_lane()) - 1ull;
}

__device__ __forceinline__ int gs_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ double gs_readlane_f64(double v, int l) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, l);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ int64_t gs_readlane_i64(int64_t v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
// f(std::integral_constant<int, n>{}) for a runtime n in [1, N] (one compare
// chain, then straight-line code specialised for n)
template <int N, class F>
__device__ __forceinline__ void gs_dispatch_upto(int n, F &&f) {
    if constexpr (N >= 1) {
        if (n >= N) {
            f(std::integral_constant<int, N>{});
            return;
        }
        gs_dispatch_upto<N - 1>(n, f);
    }
}
__device__ __forceinline__ int64_t gs_uniform64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Order-preserving maps of scores onto unsigned integers (larger score -> larger key).
__device__ __forceinline__ uint32_t gs_key_f32(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float gs_unkey_f32(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ uint64_t gs_key_f64(double d) {
    uint64_t u = (uint64_t)__double_as_longlong(d);
    return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}
__device__ __forceinline__ double gs_unkey_f64(uint64_t k) {
    uint64_t u = (k & 0x8000000000000000ull) ? (k & 0x7FFFFFFFFFFFFFFFull) : ~k;
    return __longlong_as_double((long long)u);
}

// Weight decoding by storage type.
template <int WT>
struct gs_weight;
template <>
struct gs_weight<GS_W_F32> {
    using store_t = float;
    using acc_t = float;
    using qw_t = float;
    __device__ __forceinline__ static float decode(float w) { return w; }
    __device__ __forceinline__ static float bload(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    }
};
template <>
struct gs_weight<GS_W_F16> {
    using store_t = _Float16;
    using acc_t = float;
    using qw_t = float;
    __device__ __forceinline__ static float decode(_Float16 w) { return (float)w; }
    __device__ __forceinline__ static _Float16 bload(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
    }
};
template <>
struct gs_weight<GS_W_U8> {
    using store_t = uint8_t;
    using acc_t = uint32_t;
    using qw_t = uint8_t;
    __device__ __forceinline__ static uint32_t decode(uint8_t w) { return (uint32_t)w; }
    __device__ __forceinline__ static uint8_t bload(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
    }
};

// Raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3:
// 32-bit data format, no swizzle).  Loads at offsets >= bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gs_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t gs_bload32(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint2 gs_bload64(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v[0], v[1]);
}

// Histogram bin of a score (a positive integer sum, as fp32): 64 bins per binade
// of [1, 2^32) -- the exponent above 2^0 and six mantissa bits of its fp32 value,
// bins at most 1/64 of their value wide -- which fills the 2048 bins exactly;
// values below 1 fall in bin 0, 2^32 (the fp32 image of the largest uint32) in
// the last.  Monotone in v, so a bin's lower edge bounds every value in it and
// above from below.
constexpr int GS_HIST_BINS = 2048;
__device__ __forceinline__ uint32_t gs_bin_of(float v) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t b = u < 0x3F800000u ? 0u : (u - 0x3F800000u) >> 17;
    return b < (uint32_t)(GS_HIST_BINS - 1) ? b : (uint32_t)(GS_HIST_BINS - 1);
}
__device__ __forceinline__ float gs_bin_edge(uint32_t b) { return __uint_as_float(0x3F800000u + (b << 17)); }

// Orders LDS accesses among the lanes of one wave.  The LDS executes a wave's
// instructions in order, but without a fence the compiler may move or forward
// an access across the exchange point (it assumes no other lane writes what
// this lane reads), so lanes that pass data through LDS call this in between.
__device__ __forceinline__ void gs_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-wide inclusive prefix sum of 32-bit values (lane order).
__device__ __forceinline__ uint32_t gs_wave_incl_scan(uint32_t v) {
#pragma unroll
    for (int d = 1; d < GS_WAVE; d <<= 1) {
        uint32_t o = __shfl_up(v, d, GS_WAVE);
        if (gs_lane() >= d) v += o;
    }
    return v;
}

// max over the wave's lanes (DPP row shifts and row broadcasts, no LDS)
__device__ __forceinline__ uint32_t gs_wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x113, 0xf, 0xf, false));  // row_shr:3
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x114, 0xf, 0xe, false));  // row_shr:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x118, 0xf, 0xc, false));  // row_shr:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t gs_wave_sum(uint32_t v) {
#pragma unroll
    for (int d = GS_WAVE / 2; d >= 1; d >>= 1) v += __shfl_xor(v, d, GS_WAVE);
    return v;
}

// Relaxed device-scope loads/stores of shared counters (bypass the per-CU cache).
__device__ __forceinline__ uint32_t gs_load_relaxed(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
