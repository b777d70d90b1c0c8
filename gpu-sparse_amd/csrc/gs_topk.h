// Exact top-k selection of one row per workgroup (1024 threads), shared by the
// search pipeline and the dense-row entry points.
//
// Entries expose a monotone unsigned key (larger score -> larger key) and a
// unique doc id; the order is key descending, doc ascending.  A radix select
// over 8-bit digits of the key (then of the doc id among ties at the k-th key)
// finds the cut, the k selected entries are collected into LDS and sorted with
// Batcher's bitonic network.  The sort buffer is dynamic LDS of sel_lds_bytes(k)
// (next power of two of k entries), so a small k leaves room for a second
// workgroup on the CU.
#pragma once

#include "gs_common.h"

namespace gs {

constexpr int kSelThreads = 1024;
constexpr int kMaxK = 8192;  // LDS sort capacity


// LDS of one selection: the radix state (static) ...
struct SelStatic {
    uint32_t hist[256];
    uint64_t prefix;
    uint32_t kr;
    uint32_t tie_total;
    uint32_t doc_prefix;
    uint32_t n_sel;
};
// ... and each thread's view of it plus the dynamic sort buffer (key, doc).
struct SelShared {
    SelStatic &s;
    uint64_t *key;
    uint32_t *doc;
    int cap;
};

// Sort-buffer entries for a selection of k: the next power of two (bitonic sort).
__host__ __device__ constexpr int sel_cap(int k) {
    int c = 1;
    while (c < k && c < kMaxK) c <<= 1;
    return c;
}
inline size_t sel_lds_bytes(int k) { return (size_t)sel_cap(k) * (sizeof(uint64_t) + sizeof(uint32_t)); }
// Raises a selection kernel's dynamic LDS limit when sel_lds_bytes(k) exceeds
// the 64 KiB default.
inline hipError_t sel_attr(const void *fn, size_t lds) {
    return lds > 65536 ? hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) : hipSuccess;
}

extern __shared__ __align__(16) unsigned char gs_sel_lds[];

// The view of a selection kernel launched with sel_lds_bytes(k) of dynamic LDS.
__device__ __forceinline__ SelShared sel_view(SelStatic &st, int k) {
    const int cap = sel_cap(k);
    uint64_t *key = reinterpret_cast<uint64_t *>(gs_sel_lds);
    return SelShared{st, key, reinterpret_cast<uint32_t *>(key + cap), cap};
}

// Wave-wide search of a 256-bin histogram: the digit at which the running count
// (from digit 255 down when `desc`, from 0 up otherwise) reaches kr, and the
// count of the bins before it.  Lane l holds four consecutive bins; a wave scan
// of their sums finds the lane, which walks its four.  All lanes return both.
__device__ __forceinline__ void sel_find_digit(const uint32_t *hist, uint32_t kr, bool desc, int &digit,
                                               uint32_t &before) {
    const int lane = gs_lane();
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = hist[desc ? 255 - (4 * lane + i) : 4 * lane + i];
    const uint32_t tot = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = gs_wave_incl_scan(tot);
    const uint32_t excl = incl - tot;
    const uint64_t bal = __ballot(excl < kr && kr <= incl);
    if (!bal) {  // kr beyond the total (not reached by a consistent histogram): last digit
        digit = desc ? 0 : 255;
        before = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63) - hist[digit];
        return;
    }
    const int L = __ffsll((unsigned long long)bal) - 1;
    int dg = 0;
    uint32_t cum = excl;
    if (lane == L) {
        int i = 0;
        for (; i < 3; ++i) {
            if (cum + h[i] >= kr) break;
            cum += h[i];
        }
        dg = desc ? 255 - (4 * lane + i) : 4 * lane + i;
    }
    digit = __builtin_amdgcn_readlane(dg, L);
    before = (uint32_t)__builtin_amdgcn_readlane((int)cum, L);
}

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

// Dense row (fp64 or uint32 values, doc = column) past a cutoff: only the
// entries after (ck, cd) in (key desc, doc asc) order take part, as key + 1 (a
// finite score's key is below 2^64 - 1); the others read 0, filtered out.  With
// `cut` false every entry takes part.  Successive selections of up to kMaxK
// entries, each after the previous one's last entry, give a top-k of any k.
template <bool F64>
struct SrcRowAfter {
    const void *v;
    int64_t n;
    uint64_t ck;
    uint32_t cd;
    bool cut;
    __device__ uint64_t k(int64_t i) const {
        const uint64_t kk = F64 ? gs_key_f64(reinterpret_cast<const double *>(v)[i])
                                : (uint64_t)reinterpret_cast<const uint32_t *>(v)[i];
        const bool after = !cut || kk < ck || (kk == ck && (uint32_t)i > cd);
        return after ? kk + 1 : 0;
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
        sh.s.prefix = 0;
        sh.s.kr = (uint32_t)k;
        sh.s.n_sel = 0;
        sh.s.tie_total = 0;
        sh.s.doc_prefix = 0;
    }
    __syncthreads();
    // count eligible entries
    uint32_t local = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x)
        local += !(skip_zero && src.k(i) == 0);
    local = gs_wave_sum(local);
    if (gs_lane() == 0) atomicAdd(&sh.s.n_sel, local);
    __syncthreads();
    const uint32_t n_elig = sh.s.n_sel;
    __syncthreads();
    if (threadIdx.x == 0) sh.s.n_sel = 0;
    __syncthreads();

    uint64_t kstar = 0;
    uint32_t dstar = 0xFFFFFFFFu;
    if (n_elig > (uint32_t)k) {
        // radix select of the k-th largest key, 8 bits per pass from the top
        for (int shift = KEY_BITS - 8; shift >= 0; shift -= 8) {
            for (int b = threadIdx.x; b < 256; b += blockDim.x) sh.s.hist[b] = 0;
            __syncthreads();
            const uint64_t pre = sh.s.prefix;
            const uint64_t hmask = (shift + 8 >= 64) ? 0ull : (~0ull << (shift + 8));
            for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
                const uint64_t kk = src.k(i);
                if (skip_zero && kk == 0) continue;
                if ((kk & hmask) == pre) atomicAdd(&sh.s.hist[(kk >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (threadIdx.x < 64) {
                int dg;
                uint32_t cum;
                sel_find_digit(sh.s.hist, sh.s.kr, true, dg, cum);
                if (threadIdx.x == 0) {
                    sh.s.kr -= cum;
                    sh.s.prefix = pre | ((uint64_t)dg << shift);
                    sh.s.tie_total = sh.s.hist[dg];
                }
            }
            __syncthreads();
        }
        kstar = sh.s.prefix;
        const uint32_t need = sh.s.kr;  // ties at kstar to take, by smallest doc
        if (sh.s.tie_total > need) {
            if (threadIdx.x == 0) sh.s.doc_prefix = 0;
            __syncthreads();
            for (int shift = 24; shift >= 0; shift -= 8) {
                for (int b = threadIdx.x; b < 256; b += blockDim.x) sh.s.hist[b] = 0;
                __syncthreads();
                const uint32_t pre = sh.s.doc_prefix;
                const uint32_t hmask = shift + 8 >= 32 ? 0u : (~0u << (shift + 8));
                for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
                    if (src.k(i) != kstar) continue;
                    const uint32_t dd = src.d(i);
                    if ((dd & hmask) == pre) atomicAdd(&sh.s.hist[(dd >> shift) & 255u], 1u);
                }
                __syncthreads();
                if (threadIdx.x < 64) {
                    int dg;
                    uint32_t cum;
                    sel_find_digit(sh.s.hist, sh.s.kr, false, dg, cum);
                    if (threadIdx.x == 0) {
                        sh.s.kr -= cum;
                        sh.s.doc_prefix = pre | ((uint32_t)dg << shift);
                    }
                }
                __syncthreads();
            }
            dstar = sh.s.doc_prefix;
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
            const uint32_t s = atomicAdd(&sh.s.n_sel, 1u);
            if (s < (uint32_t)sh.cap) {
                sh.key[s] = kk;
                sh.doc[s] = src.d(i);
            }
        }
    }
    __syncthreads();
    int c = (int)sh.s.n_sel;
    if (c > sh.cap) c = sh.cap;
    __syncthreads();
    block_sort(sh, c);
    return c;
}


}  // namespace gs
