// Exact top-k selection of one row per workgroup (1024 threads), shared by the
// search pipeline and the dense-row entry points.
//
// Entries expose a monotone unsigned key (larger score -> larger key) and a
// unique doc id; the order is key descending, doc ascending.  A radix select
// over 8-bit digits of the key (then of the doc id among ties at the k-th key)
// finds the cut, the k selected entries are collected into LDS and sorted with
// Batcher's bitonic network.
#pragma once

#include "gs_common.h"

namespace gs {

constexpr int kSelThreads = 1024;
constexpr int kMaxK = 8192;  // LDS sort capacity


struct SelShared {
    uint64_t key[kMaxK];
    uint32_t doc[kMaxK];
    uint32_t hist[256];
    uint64_t prefix;
    uint32_t kr;
    uint32_t tie_total;
    uint32_t doc_prefix;
    uint32_t n_sel;
};

// Entries of a selection source expose a monotone key and a unique doc id.
struct SrcCand32 {  // candidate list with 32-bit keys
    const uint32_t *key;
    const uint32_t *doc;
    int64_t n;
    __device__ uint64_t k(int64_t i) const { return key[i]; }
    __device__ uint32_t d(int64_t i) const { return doc[i]; }
};
struct SrcCand64 {  // rescored list with 64-bit keys
    const uint64_t *key;
    const uint32_t *doc;
    int64_t n;
    __device__ uint64_t k(int64_t i) const { return key[i]; }
    __device__ uint32_t d(int64_t i) const { return doc[i]; }
};
struct SrcRowF64 {  // dense fp64 row, doc = column
    const double *v;
    int64_t n;
    __device__ uint64_t k(int64_t i) const { return gs_key_f64(v[i]); }
    __device__ uint32_t d(int64_t i) const { return (uint32_t)i; }
};
struct SrcRowU32 {
    const uint32_t *v;
    int64_t n;
    __device__ uint64_t k(int64_t i) const { return v[i]; }
    __device__ uint32_t d(int64_t i) const { return (uint32_t)i; }
};
struct SrcCandF32 {  // compacted (column, fp32 value) candidates
    const float *val;
    const int32_t *idx;
    int64_t n;
    __device__ uint64_t k(int64_t i) const { return gs_key_f32(val[i]); }
    __device__ uint32_t d(int64_t i) const { return (uint32_t)idx[i]; }
};
struct SrcRowF32 {  // dense fp32 row, optionally only entries >= tau
    const float *v;
    int64_t n;
    uint32_t min_key;
    __device__ uint64_t k(int64_t i) const {
        const uint32_t kk = gs_key_f32(v[i]);
        return kk >= min_key ? (uint64_t)kk + 1 : 0;  // 0 = filtered out
    }
    __device__ uint32_t d(int64_t i) const { return (uint32_t)i; }
};

__device__ __forceinline__ bool sel_before(uint64_t ka, uint32_t da, uint64_t kb, uint32_t db) {
    return ka > kb || (ka == kb && da < db);
}

// Bitonic sort of sh.key/sh.doc[0, n) into (key desc, doc asc).
__device__ void block_sort(SelShared &sh, int n) {
    int np = 1;
    while (np < n) np <<= 1;
    for (int i = n + threadIdx.x; i < np; i += blockDim.x) {
        sh.key[i] = 0;
        sh.doc[i] = 0xFFFFFFFFu;
    }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t kl = sh.key[lo], kh = sh.key[hi];
                const uint32_t dl = sh.doc[lo], dh = sh.doc[hi];
                const bool hi_first = sel_before(kh, dh, kl, dl);
                if (up == hi_first) {
                    sh.key[lo] = kh;
                    sh.key[hi] = kl;
                    sh.doc[lo] = dh;
                    sh.doc[hi] = dl;
                }
            }
            __syncthreads();
        }
    }
}

// Exact top-k of a source by (key desc, doc asc).  Keys equal to 0 are ignored
// when `skip_zero` (used by filtered sources).  Returns the number selected
// (min(k, #entries)), sorted in sh.key/sh.doc.  KEY_BITS: 32 or 64.
template <int KEY_BITS, class Src>
__device__ int block_topk(const Src &src, int k, SelShared &sh, bool skip_zero) {
    const int64_t n = src.n;
    if (threadIdx.x == 0) {
        sh.prefix = 0;
        sh.kr = (uint32_t)k;
        sh.n_sel = 0;
        sh.tie_total = 0;
        sh.doc_prefix = 0;
    }
    __syncthreads();
    // count eligible entries
    uint32_t local = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x)
        local += !(skip_zero && src.k(i) == 0);
    local = gs_wave_sum(local);
    if (gs_lane() == 0) atomicAdd(&sh.n_sel, local);
    __syncthreads();
    const uint32_t n_elig = sh.n_sel;
    __syncthreads();
    if (threadIdx.x == 0) sh.n_sel = 0;
    __syncthreads();

    uint64_t kstar = 0;
    uint32_t dstar = 0xFFFFFFFFu;
    if (n_elig > (uint32_t)k) {
        // radix select of the k-th largest key, 8 bits per pass from the top
        for (int shift = KEY_BITS - 8; shift >= 0; shift -= 8) {
            for (int b = threadIdx.x; b < 256; b += blockDim.x) sh.hist[b] = 0;
            __syncthreads();
            const uint64_t pre = sh.prefix;
            const uint64_t hmask = (shift + 8 >= 64) ? 0ull : (~0ull << (shift + 8));
            for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
                const uint64_t kk = src.k(i);
                if (skip_zero && kk == 0) continue;
                if ((kk & hmask) == pre) atomicAdd(&sh.hist[(kk >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                uint32_t kr = sh.kr, cum = 0;
                int dg = 255;
                for (; dg > 0; --dg) {
                    if (cum + sh.hist[dg] >= kr) break;
                    cum += sh.hist[dg];
                }
                sh.kr = kr - cum;
                sh.prefix = pre | ((uint64_t)dg << shift);
                sh.tie_total = sh.hist[dg];
            }
            __syncthreads();
        }
        kstar = sh.prefix;
        const uint32_t need = sh.kr;  // ties at kstar to take, by smallest doc
        if (sh.tie_total > need) {
            if (threadIdx.x == 0) sh.doc_prefix = 0;
            __syncthreads();
            for (int shift = 24; shift >= 0; shift -= 8) {
                for (int b = threadIdx.x; b < 256; b += blockDim.x) sh.hist[b] = 0;
                __syncthreads();
                const uint32_t pre = sh.doc_prefix;
                const uint32_t hmask = shift + 8 >= 32 ? 0u : (~0u << (shift + 8));
                for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
                    if (src.k(i) != kstar) continue;
                    const uint32_t dd = src.d(i);
                    if ((dd & hmask) == pre) atomicAdd(&sh.hist[(dd >> shift) & 255u], 1u);
                }
                __syncthreads();
                if (threadIdx.x == 0) {
                    uint32_t kr = sh.kr, cum = 0;
                    int dg = 0;
                    for (; dg < 255; ++dg) {
                        if (cum + sh.hist[dg] >= kr) break;
                        cum += sh.hist[dg];
                    }
                    sh.kr = kr - cum;
                    sh.doc_prefix = pre | ((uint32_t)dg << shift);
                }
                __syncthreads();
            }
            dstar = sh.doc_prefix;
        }
    }
    const bool all = n_elig <= (uint32_t)k;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t kk = src.k(i);
        if (skip_zero && kk == 0) continue;
        bool take = all;
        if (!all) {
            if (kk > kstar)
                take = true;
            else if (kk == kstar)
                take = src.d(i) <= dstar;
        }
        if (take) {
            const uint32_t s = atomicAdd(&sh.n_sel, 1u);
            if (s < (uint32_t)kMaxK) {
                sh.key[s] = kk;
                sh.doc[s] = src.d(i);
            }
        }
    }
    __syncthreads();
    int c = (int)sh.n_sel;
    if (c > kMaxK) c = kMaxK;
    __syncthreads();
    block_sort(sh, c);
    return c;
}


}  // namespace gs
