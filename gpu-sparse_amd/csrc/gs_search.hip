// Exact batched SPLADE scoring and top-k selection for gfx950.
//
// What is computed is the reference's scatter-add (src/triton_kernel.py:93-156):
//     score[q, d] = sum over valid terms j of q_w[q, j] * w(q_t[q, j], d)
// followed by an exact top-k (torch.topk at triton_kernel.py:199, or the
// chunked / threshold-compacted selection of src/fused_topk.py:106-160).
//
// How it is computed here:
//  * Documents are cut into tiles of 2^tile_log2 docs.  One wave owns one
//    (query, tile) pair and accumulates that query's scores for the tile in a
//    private LDS slice with ds_add, walking the query's terms in order and, per
//    term, only the postings inside the tile (per-(term, tile) bounds).  No
//    [B, N] accumulator exists and no global atomics are issued for scores.
//  * Workgroups are mapped tile-major and XCD-aware, so the waves resident on an
//    XCD work on the same tiles and share posting lines in that XCD's L2.
//  * Selection is fused into the scoring kernel.  A dense sample of the first
//    tiles seeds a per-query lower bound tau on the k-th score; every wave then
//    emits only docs scoring >= tau - margin (ballot compaction, one atomic per
//    64 docs), counts them in a per-query histogram of score bins and raises tau
//    from that histogram.  tau never exceeds the true k-th score, so no doc of
//    the answer is dropped.
//  * Float configurations accumulate fp32 in the tiles.  The fp32 k-th score
//    tau' and a rigorous error bound E pick every doc whose fp64 score can reach
//    the top k (fp32 >= tau' - 2E); those are rescored in fp64 in query-term
//    order (exactly the fp64 scatter-add), and the final order is
//    (score desc, doc asc).  uint8 configurations sum exactly in uint32.
//  * A row whose candidates overflow, or that has fewer than k positive docs,
//    is flagged and finished by the dense path (fp64 / uint32 tiles written to
//    a full row, then an exact radix select).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gs_common.h"

namespace {

constexpr int kSelThreads = 1024;
constexpr int kMaxK = 8192;          // LDS sort capacity of the selection kernels
constexpr int kRescoreCap = 16384;   // candidates rescored per query before the dense fallback
constexpr int kDefaultSample = 16;
constexpr int kDefaultCandCap = 65536;
constexpr size_t kTileLds = 128 * 1024;  // LDS budget of a scoring workgroup

enum ScoreMode { kDense = 0, kDense64 = 1, kEmit = 2 };

template <class T>
__global__ void k_fill(T *p, int64_t n, T v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// ---------------------------------------------------------------------- per-query prep

// Error bound of the fp32 tile scores.  A doc's fp32 score is a sum of at most
// n = sum_j (1 + dup[t_j]) rounded products, so |fp32 - exact| <= g32(2n) * M and
// |fp64 - exact| <= g64(2n) * M with M = sum_j |q_j| * max|w(t_j)| * (1 + dup[t_j]),
// g(m) = m*u / (1 - m*u).  The candidates needed are those with
// fp32 >= tau' - margin, margin = 2 * (g32 + g64) * M (slightly inflated).
template <int WT>
__global__ void k_query_prep(const int32_t *__restrict__ qt, const void *__restrict__ qw, int32_t B,
                             int32_t T, int32_t V, const float *__restrict__ max_abs,
                             const int32_t *__restrict__ dup, double *__restrict__ margin,
                             uint32_t *__restrict__ tau, uint32_t *__restrict__ cnt,
                             uint32_t *__restrict__ maxbin) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= B) return;
    double M = 0.0, n = 0.0;
    for (int j = 0; j < T; ++j) {
        const int32_t t = qt[(int64_t)q * T + j];
        if ((uint32_t)t >= (uint32_t)V) continue;
        const double m = 1.0 + (double)dup[t];
        double wq;
        if (WT == GS_W_U8)
            wq = (double)reinterpret_cast<const uint8_t *>(qw)[(int64_t)q * T + j];
        else
            wq = fabs((double)reinterpret_cast<const float *>(qw)[(int64_t)q * T + j]);
        M += wq * (double)max_abs[t] * m;
        n += m;
    }
    const double m2 = 2.0 * n + 2.0;
    const double u32 = 0x1p-24, u64 = 0x1p-53;
    const double g32 = m2 * u32 / (1.0 - m2 * u32);
    const double g64 = m2 * u64 / (1.0 - m2 * u64);
    margin[q] = WT == GS_W_U8 ? 0.0 : 2.0 * (g32 + g64) * M * (1.0 + 1e-9);
    tau[q] = 0;
    cnt[q] = 0;
    maxbin[q] = 0;
}

// ---------------------------------------------------------------------- tile scoring

struct ScoreArgs {
    const int32_t *doc;
    const void *w;
    const int64_t *offsets;
    const int32_t *tb;  // [V][n_tiles + 1]
    const int32_t *qt;
    const void *qw;
    const int32_t *rows;  // optional row -> query map
    int64_t n_docs;
    int32_t V, T, R, tile_log2, n_tiles;
    int32_t tile_begin, tiles, groups, per_xcd;
    // dense output
    void *dense;
    int64_t dense_ld, dense_col0;
    // emission
    uint32_t *tau, *cnt, *maxbin, *hist, *cand_doc, *cand_key;
    const double *margin;
    int32_t cap, k;
};

template <class A>
__device__ __forceinline__ void lds_add(A *p, A v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Largest float <= (tau - margin) as a threshold for fp32 scores.
__device__ __forceinline__ float lowered_threshold(uint32_t tau_bits, double margin) {
    const double t = (double)__uint_as_float(tau_bits) - margin;
    return __double2float_rd(t);
}

// Lower bound on uint32 scores whose fp32 image lies in bins >= b.
__device__ __forceinline__ uint32_t int_threshold_of_bin(uint32_t b) {
    const double e = (double)gs_bin_edge(b);
    return (uint32_t)floor(e / (1.0 + 0x1p-23));
}

// Recompute tau[q] from the histogram (bins >= top scanned downward): the lower
// edge of the highest bin b with count(bins >= b) >= k.  Whole wave calls it.
template <bool FP>
__device__ void raise_tau(uint32_t *tau, const uint32_t *hist, uint32_t top, int k) {
    const int lane = gs_lane();
    const uint32_t cur = gs_load_relaxed(tau);
    const uint32_t cur_bin = FP ? (cur >> 20) : gs_bin_of((float)cur);
    uint32_t cum = 0;
    for (int b = (int)top; b >= 0 && b + 1 > (int)cur_bin; b -= 64) {
        const int bb = b - lane;
        const uint32_t c = bb >= 0 ? gs_load_relaxed(hist + bb) : 0u;
        const uint32_t inc = gs_wave_incl_scan(c);
        const uint64_t hit = __ballot(cum + inc >= (uint32_t)k);
        if (hit) {
            const int l = __ffsll((unsigned long long)hit) - 1;
            const uint32_t bin = (uint32_t)(b - l);
            if (lane == 0 && bin > cur_bin) {
                const uint32_t key = FP ? (bin << 20) : int_threshold_of_bin(bin);
                atomicMax(tau, key);
            }
            return;
        }
        cum += __shfl(inc, 63, 64);
    }
}

template <int WT, int MODE, int UNROLL>
__global__ void __launch_bounds__(512) k_score_tiles(const ScoreArgs a) {
    using W = gs_weight<WT>;
    using store_t = typename W::store_t;
    using acc32_t = typename W::acc_t;
    constexpr bool kF64 = MODE == kDense64 && WT != GS_W_U8;
    using acc_t = typename std::conditional<kF64, double, acc32_t>::type;
    constexpr bool FP = WT != GS_W_U8;

    extern __shared__ __align__(16) unsigned char lds_raw[];
    const int waves = (int)(blockDim.x >> 6);
    const int wave = gs_uniform((int)(threadIdx.x >> 6));
    const int lane = gs_lane();

    // XCD-aware block order: workgroup i runs on XCD i % 8; give each XCD a
    // contiguous run of (tile, query group) pairs, query groups fastest.
    const int64_t lin = (int64_t)(blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
    if (lin >= (int64_t)a.tiles * a.groups) return;
    const int tile = a.tile_begin + (int)(lin / a.groups);
    const int r = (int)(lin % a.groups) * waves + wave;
    if (r >= a.R) return;
    const int q = a.rows ? gs_uniform(a.rows[r]) : r;

    const int TILE = 1 << a.tile_log2;
    acc_t *acc = reinterpret_cast<acc_t *>(lds_raw) + (size_t)wave * TILE;
    for (int i = lane; i < TILE; i += 64) acc[i] = (acc_t)0;

    const int64_t doc0 = (int64_t)tile << a.tile_log2;
    const int32_t *qt = a.qt + (int64_t)q * a.T;
    const int64_t row = (int64_t)a.n_tiles + 1;
    const store_t *wall = reinterpret_cast<const store_t *>(a.w);
    for (int j = 0; j < a.T; ++j) {
        const int32_t t = qt[j];
        if ((uint32_t)t >= (uint32_t)a.V) continue;
        const int32_t *bt = a.tb + (int64_t)t * row + tile;
        const int lo = bt[0], hi = bt[1];
        if (lo >= hi) continue;
        const int64_t base = a.offsets[t];
        const int32_t *dp = a.doc + base;
        const store_t *wp = wall + base;
        // contribution of one posting: fp32 (or fp64 for the dense fp64 rows) product,
        // exact uint32 product for uint8 impacts
        acc_t wq;
        if (FP)
            wq = (acc_t) reinterpret_cast<const float *>(a.qw)[(int64_t)q * a.T + j];
        else
            wq = (acc_t) reinterpret_cast<const uint8_t *>(a.qw)[(int64_t)q * a.T + j];
        auto contrib = [&](store_t wv) -> acc_t {
            if (kF64) return wq * (acc_t)W::decode(wv);
            if (FP) return (acc_t)((float)wq * (float)W::decode(wv));
            return (acc_t)((uint32_t)wq * (uint32_t)W::decode(wv));
        };
        int p = lo + lane;
        // full blocks of 64*UNROLL postings: branch-free, all loads in flight together
        const int nfull = (hi - lo) / (64 * UNROLL);
        for (int it = 0; it < nfull; ++it, p += 64 * UNROLL) {
            int32_t d[UNROLL];
            store_t wv[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                d[u] = dp[p + 64 * u];
                wv[u] = wp[p + 64 * u];
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) lds_add<acc_t>(acc + (int)(d[u] - doc0), contrib(wv[u]));
        }
        for (; p < hi; p += 64) lds_add<acc_t>(acc + (int)(dp[p] - doc0), contrib(wp[p]));
    }

    const int64_t left = a.n_docs - doc0;
    const int ncols = left < TILE ? (int)left : TILE;

    if (MODE != kEmit) {
        acc_t *out = reinterpret_cast<acc_t *>(a.dense) + (int64_t)r * a.dense_ld + (doc0 - a.dense_col0);
        for (int i = lane; i < ncols; i += 64) out[i] = acc[i];
        return;
    }

    // ---- emission of candidates >= lowered tau
    uint32_t *tau = a.tau + q;
    const uint32_t tau_now = gs_load_relaxed(tau);
    float thr_f = 0.0f;
    uint32_t thr_u = 0;
    if (FP)
        thr_f = lowered_threshold(tau_now, a.margin[q]);
    else
        thr_u = tau_now;
    uint32_t *hist = a.hist + (int64_t)q * GS_HIST_BINS;
    uint32_t *cdoc = a.cand_doc + (int64_t)q * a.cap;
    uint32_t *ckey = a.cand_key + (int64_t)q * a.cap;
    uint32_t max_bin = 0;
    bool any = false;
    for (int i0 = 0; i0 < ncols; i0 += 64) {
        const int i = i0 + lane;
        bool keep = false;
        uint32_t key = 0;
        float fv = 0.0f;
        if (i < ncols) {
            const acc_t v = acc[i];
            if (FP) {
                fv = (float)v;
                keep = fv > 0.0f && fv >= thr_f;
                key = __float_as_uint(fv);
            } else {
                key = (uint32_t)v;
                keep = key > 0u && key >= thr_u;
                fv = (float)key;
            }
        }
        const uint64_t m = __ballot(keep);
        if (m == 0) continue;
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(a.cnt + q, (uint32_t)__popcll(m));
        base = __shfl(base, 0, 64);
        if (keep) {
            const uint32_t slot = base + (uint32_t)__popcll(m & gs_lanemask_lt());
            if (slot < (uint32_t)a.cap) {
                cdoc[slot] = (uint32_t)(doc0 + i);
                ckey[slot] = key;
            }
            const uint32_t b = gs_bin_of(fv);
            atomicAdd(hist + b, 1u);
            max_bin = b > max_bin ? b : max_bin;
        }
        any = true;
    }
    if (!any) return;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const uint32_t o = __shfl_xor(max_bin, d, 64);
        max_bin = o > max_bin ? o : max_bin;
    }
    uint32_t top = 0;
    if (lane == 0) top = atomicMax(a.maxbin + q, max_bin);
    top = __shfl(top, 0, 64);
    top = top > max_bin ? top : max_bin;
    raise_tau<FP>(tau, hist, top, a.k);
}

// ---------------------------------------------------------------------- seeding

// Per query: tau from the histogram of the dense sample, then emission of the
// sample's candidates exactly as the scoring kernel would emit them.
template <int WT>
__global__ void __launch_bounds__(1024) k_seed(const void *__restrict__ sample, int64_t ld, int64_t ncols,
                                               int32_t k, const double *__restrict__ margin,
                                               uint32_t *__restrict__ tau_arr, uint32_t *__restrict__ cnt,
                                               uint32_t *__restrict__ maxbin, uint32_t *__restrict__ hist_all,
                                               uint32_t *__restrict__ cand_doc, uint32_t *__restrict__ cand_key,
                                               int32_t cap) {
    constexpr bool FP = WT != GS_W_U8;
    using acc_t = typename gs_weight<WT>::acc_t;
    __shared__ uint32_t h[GS_HIST_BINS];
    __shared__ uint32_t s_tau, s_maxbin;
    const int q = blockIdx.x;
    const acc_t *row = reinterpret_cast<const acc_t *>(sample) + (int64_t)q * ld;
    for (int b = threadIdx.x; b < GS_HIST_BINS; b += blockDim.x) h[b] = 0;
    if (threadIdx.x == 0) {
        s_tau = 0;
        s_maxbin = 0;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < ncols; i += blockDim.x) {
        const acc_t v = row[i];
        if (v > (acc_t)0) atomicAdd(&h[gs_bin_of((float)v)], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        uint32_t cum = 0;
        for (int b = GS_HIST_BINS - 1; b >= 0; b -= 64) {
            const int bb = b - gs_lane();
            const uint32_t c = bb >= 0 ? h[bb] : 0u;
            const uint32_t inc = gs_wave_incl_scan(c);
            const uint64_t hit = __ballot(cum + inc >= (uint32_t)k);
            if (hit) {
                const uint32_t bin = (uint32_t)(b - (__ffsll((unsigned long long)hit) - 1));
                if (gs_lane() == 0) s_tau = FP ? (bin << 20) : int_threshold_of_bin(bin);
                break;
            }
            cum += __shfl(inc, 63, 64);
        }
    }
    __syncthreads();
    const uint32_t tau = s_tau;
    float thr_f = 0.0f;
    uint32_t thr_u = tau;
    if (FP) thr_f = lowered_threshold(tau, margin[q]);
    uint32_t *hist = hist_all + (int64_t)q * GS_HIST_BINS;
    uint32_t max_bin = 0;
    const int lane = gs_lane();
    const int64_t span = (ncols + 63) & ~int64_t(63);
    for (int64_t i = threadIdx.x; i < span; i += blockDim.x) {
        bool keep = false;
        uint32_t key = 0;
        float fv = 0.0f;
        if (i < ncols) {
            const acc_t v = row[i];
            if (FP) {
                fv = (float)v;
                keep = fv > 0.0f && fv >= thr_f;
                key = __float_as_uint(fv);
            } else {
                key = (uint32_t)v;
                keep = key > 0u && key >= thr_u;
                fv = (float)key;
            }
        }
        const uint64_t m = __ballot(keep);
        if (m == 0) continue;
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(cnt + q, (uint32_t)__popcll(m));
        base = __shfl(base, 0, 64);
        if (keep) {
            const uint32_t slot = base + (uint32_t)__popcll(m & gs_lanemask_lt());
            if (slot < (uint32_t)cap) {
                cand_doc[(int64_t)q * cap + slot] = (uint32_t)i;
                cand_key[(int64_t)q * cap + slot] = key;
            }
            const uint32_t b = gs_bin_of(fv);
            atomicAdd(hist + b, 1u);
            max_bin = b > max_bin ? b : max_bin;
        }
    }
    atomicMax(&s_maxbin, max_bin);
    __syncthreads();
    if (threadIdx.x == 0) {
        tau_arr[q] = tau;
        maxbin[q] = s_maxbin;
    }
}

// ---------------------------------------------------------------------- block top-k

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

// ---------------------------------------------------------------------- candidate selection

// Float rows: fp32 k-th tau' -> collect every candidate >= tau' - margin for
// rescoring.  Integer rows: final top-k written directly.
template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_cands(const uint32_t *__restrict__ cand_doc, const uint32_t *__restrict__ cand_key,
                   const uint32_t *__restrict__ cnt, int32_t cap, int32_t k, const double *__restrict__ margin,
                   uint32_t *__restrict__ resc_doc, uint32_t *__restrict__ resc_cnt, int32_t resc_cap,
                   void *__restrict__ out_scores, int64_t *__restrict__ out_ids, int32_t *__restrict__ status) {
    constexpr bool FP = WT != GS_W_U8;
    __shared__ SelShared sh;
    __shared__ uint32_t s_m;
    const int q = blockIdx.x;
    const uint32_t n = cnt[q];
    if (n > (uint32_t)cap || n < (uint32_t)k) {
        if (threadIdx.x == 0) {
            status[q] = GS_ROW_DENSE;
            if (FP) resc_cnt[q] = 0;
        }
        return;
    }
    SrcCand32 src{cand_key + (int64_t)q * cap, cand_doc + (int64_t)q * cap, (int64_t)n};
    const int c = block_topk<32>(src, k, sh, false);
    if (!FP) {
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            reinterpret_cast<int32_t *>(out_scores)[(int64_t)q * k + i] = (int32_t)sh.key[i];
            out_ids[(int64_t)q * k + i] = (int64_t)sh.doc[i];
        }
        if (threadIdx.x == 0) status[q] = GS_ROW_DONE;
        return;
    }
    (void)c;
    const float kth = __uint_as_float((uint32_t)sh.key[k - 1]);
    const float t_low = __double2float_rd((double)kth - margin[q]);
    if (!(t_low > 0.0f)) {
        if (threadIdx.x == 0) {
            status[q] = GS_ROW_DENSE;
            resc_cnt[q] = 0;
        }
        return;
    }
    if (threadIdx.x == 0) s_m = 0;
    __syncthreads();
    const uint32_t tk = __float_as_uint(t_low);
    const uint32_t *ck = cand_key + (int64_t)q * cap;
    const uint32_t *cd = cand_doc + (int64_t)q * cap;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        if (ck[i] >= tk) {
            const uint32_t s = atomicAdd(&s_m, 1u);
            if (s < (uint32_t)resc_cap) resc_doc[(int64_t)q * resc_cap + s] = cd[i];
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t m = s_m;
        if (m > (uint32_t)resc_cap) {
            status[q] = GS_ROW_DENSE;
            resc_cnt[q] = 0;
        } else {
            status[q] = GS_ROW_DONE;
            resc_cnt[q] = m;
        }
    }
}

// Exact fp64 score of (query, doc) candidates, summed in query-term order.
template <int WT>
__global__ void __launch_bounds__(256)
    k_rescore(const int32_t *__restrict__ doc_ids, const void *__restrict__ w, const int64_t *__restrict__ offsets,
              const int32_t *__restrict__ tb, int32_t V, int32_t n_tiles, int32_t tile_log2,
              const int32_t *__restrict__ qt, const float *__restrict__ qw, int32_t T,
              const uint32_t *__restrict__ resc_doc, const uint32_t *__restrict__ resc_cnt, int32_t resc_cap,
              uint64_t *__restrict__ resc_key) {
    using store_t = typename gs_weight<WT>::store_t;
    const int q = blockIdx.y;
    const uint32_t m = resc_cnt[q];
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m) return;
    const int32_t d = (int32_t)resc_doc[(int64_t)q * resc_cap + i];
    const int tile = d >> tile_log2;
    const int64_t row = (int64_t)n_tiles + 1;
    const store_t *wall = reinterpret_cast<const store_t *>(w);
    double s = 0.0;
    for (int j = 0; j < T; ++j) {
        const int32_t t = qt[(int64_t)q * T + j];
        if ((uint32_t)t >= (uint32_t)V) continue;
        const int32_t *bt = tb + (int64_t)t * row + tile;
        int lo = bt[0];
        const int hi = bt[1];
        if (lo >= hi) continue;
        const int64_t base = offsets[t];
        const int32_t *dp = doc_ids + base;
        int len = hi - lo;
        while (len > 0) {
            const int half = len >> 1;
            if (dp[lo + half] < d) {
                lo += half + 1;
                len -= half + 1;
            } else {
                len = half;
            }
        }
        const double wq = (double)qw[(int64_t)q * T + j];
        for (int p = lo; p < hi && dp[p] == d; ++p) s += wq * (double)gs_weight<WT>::decode(wall[base + p]);
    }
    resc_key[(int64_t)q * resc_cap + i] = gs_key_f64(s);
}

template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_final(const uint32_t *__restrict__ resc_doc, const uint64_t *__restrict__ resc_key,
                   const uint32_t *__restrict__ resc_cnt, int32_t resc_cap, int32_t k,
                   const int32_t *__restrict__ status, float *__restrict__ out_scores,
                   int64_t *__restrict__ out_ids) {
    __shared__ SelShared sh;
    const int q = blockIdx.x;
    if (status[q] != GS_ROW_DONE) return;
    SrcCand64 src{resc_key + (int64_t)q * resc_cap, resc_doc + (int64_t)q * resc_cap, (int64_t)resc_cnt[q]};
    block_topk<64>(src, k, sh, false);
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        out_scores[(int64_t)q * k + i] = (float)gs_unkey_f64(sh.key[i]);
        out_ids[(int64_t)q * k + i] = (int64_t)sh.doc[i];
    }
}

// Dense rows (fp64 or uint32) -> exact top-k.
template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_dense(const void *__restrict__ dense, int64_t ld, int64_t n_docs, int32_t k,
                   const int32_t *__restrict__ rows, int32_t r0, void *__restrict__ out_scores,
                   int64_t *__restrict__ out_ids) {
    __shared__ SelShared sh;
    const int r = blockIdx.x;
    const int q = rows ? rows[r0 + r] : r0 + r;
    if (WT == GS_W_U8) {
        SrcRowU32 src{reinterpret_cast<const uint32_t *>(dense) + (int64_t)r * ld, n_docs};
        block_topk<32>(src, k, sh, false);
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            reinterpret_cast<int32_t *>(out_scores)[(int64_t)q * k + i] = (int32_t)sh.key[i];
            out_ids[(int64_t)q * k + i] = (int64_t)sh.doc[i];
        }
    } else {
        SrcRowF64 src{reinterpret_cast<const double *>(dense) + (int64_t)r * ld, n_docs};
        block_topk<64>(src, k, sh, false);
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            reinterpret_cast<float *>(out_scores)[(int64_t)q * k + i] = (float)gs_unkey_f64(sh.key[i]);
            out_ids[(int64_t)q * k + i] = (int64_t)sh.doc[i];
        }
    }
}

// ---------------------------------------------------------------------- compacted top-k

// Candidates v >= tau[b] of a [B, L] fp32 matrix: one atomic slot reservation
// per 64 entries (wave ballot), as _compact_above_threshold_kernel does per block.
__global__ void __launch_bounds__(256)
    k_compact(const float *__restrict__ scores, int64_t ld, int64_t L, const float *__restrict__ tau,
              int32_t *__restrict__ cidx, float *__restrict__ cval, int32_t *__restrict__ counts,
              int32_t max_cand) {
    const int b = blockIdx.y;
    const float t = tau[b];
    const int lane = gs_lane();
    const float *row = scores + (int64_t)b * ld;
    for (int64_t i0 = (blockIdx.x * (int64_t)blockDim.x + (threadIdx.x & ~63)); i0 < L;
         i0 += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = i0 + lane;
        float v = 0.0f;
        bool keep = false;
        if (i < L) {
            v = row[i];
            keep = v >= t;
        }
        const uint64_t m = __ballot(keep);
        if (m == 0) continue;
        int32_t base = 0;
        if (lane == 0) base = atomicAdd(counts + b, (int32_t)__popcll(m));
        base = __shfl(base, 0, 64);
        if (keep) {
            const int32_t slot = base + (int32_t)__popcll(m & gs_lanemask_lt());
            if (slot < max_cand) {
                cidx[(int64_t)b * max_cand + slot] = (int32_t)i;
                cval[(int64_t)b * max_cand + slot] = v;
            }
        }
    }
}

__global__ void __launch_bounds__(kSelThreads)
    k_select_compacted(const float *__restrict__ scores, int64_t ld, int64_t L, const float *__restrict__ tau,
                       const int32_t *__restrict__ cidx, const float *__restrict__ cval,
                       const int32_t *__restrict__ counts, int32_t max_cand, int32_t k, float *__restrict__ out_v,
                       int64_t *__restrict__ out_i) {
    __shared__ SelShared sh;
    const int b = blockIdx.x;
    const int32_t cnt = counts ? counts[b] : (int32_t)0x7FFFFFFF;
    if (tau && cnt <= max_cand) {
        SrcCandF32 src{cval + (int64_t)b * max_cand, cidx + (int64_t)b * max_cand, (int64_t)cnt};
        const int c = block_topk<32>(src, k, sh, false);
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            const bool ok = i < c;
            out_v[(int64_t)b * k + i] = ok ? gs_unkey_f32((uint32_t)sh.key[i]) : -INFINITY;
            out_i[(int64_t)b * k + i] = ok ? (int64_t)sh.doc[i] : 0;
        }
    } else {
        // overflowed (or unthresholded) row: select from the full row, keys shifted by
        // one so that 0 marks entries below tau
        SrcRowF32 src{scores + (int64_t)b * ld, L, tau ? gs_key_f32(tau[b]) : 0u};
        const int c = block_topk<40>(src, k, sh, true);
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            const bool ok = i < c;
            out_v[(int64_t)b * k + i] = ok ? gs_unkey_f32((uint32_t)(sh.key[i] - 1)) : -INFINITY;
            out_i[(int64_t)b * k + i] = ok ? (int64_t)sh.doc[i] : 0;
        }
    }
}

// ---------------------------------------------------------------------- reference atomic scatter

template <int WT>
__global__ void __launch_bounds__(256)
    k_scatter_atomic(const int32_t *__restrict__ doc, const void *__restrict__ w, const int64_t *__restrict__ offsets,
                     const int32_t *__restrict__ lengths, const int64_t *__restrict__ lo_arr,
                     const int64_t *__restrict__ hi_arr, const int32_t *__restrict__ qt, const void *__restrict__ qw,
                     int32_t T, int32_t V, void *__restrict__ out, int64_t c0, int64_t clen, int64_t stride) {
    using W = gs_weight<WT>;
    const int q = blockIdx.x / T;
    const int j = blockIdx.x % T;
    const int32_t t = qt[(int64_t)q * T + j];
    if ((uint32_t)t >= (uint32_t)V) return;
    int64_t lo, hi;
    if (lo_arr) {
        lo = lo_arr[t];
        hi = hi_arr[t];
    } else {
        lo = offsets[t];
        hi = lo + lengths[t];
    }
    const typename W::store_t *wp = reinterpret_cast<const typename W::store_t *>(w);
    for (int64_t p = lo + blockIdx.y * (int64_t)blockDim.x + threadIdx.x; p < hi;
         p += (int64_t)gridDim.y * blockDim.x) {
        const int32_t d = doc[p];
        const int64_t col = (int64_t)d - c0;
        if (d < 0 || col < 0 || col >= clen) continue;
        if (WT == GS_W_U8) {
            const uint32_t wq = reinterpret_cast<const uint8_t *>(qw)[(int64_t)q * T + j];
            atomicAdd(reinterpret_cast<uint32_t *>(out) + (int64_t)q * stride + col, wq * (uint32_t)wp[p]);
        } else {
            const float wq = reinterpret_cast<const float *>(qw)[(int64_t)q * T + j];
            unsafeAtomicAdd(reinterpret_cast<float *>(out) + (int64_t)q * stride + col,
                            wq * (float)W::decode(wp[p]));
        }
    }
}

// ---------------------------------------------------------------------- host plumbing

int score_waves(int tile_log2, size_t acc_bytes) {
    const size_t per = (size_t(1) << tile_log2) * acc_bytes;
    int w = (int)(kTileLds / per);
    if (w > 8) w = 8;
    return w;
}

template <int WT, int MODE, int UNROLL>
int launch_score_u(ScoreArgs a, int waves, size_t acc_bytes, hipStream_t s) {
    static std::atomic<bool> attr_set{false};
    auto fn = k_score_tiles<WT, MODE, UNROLL>;
    const size_t lds = (size_t)waves * (size_t(1) << a.tile_log2) * acc_bytes;
    if (!attr_set.load()) {
        GS_CHECK_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)(160 * 1024)));
        attr_set.store(true);
    }
    a.groups = (a.R + waves - 1) / waves;
    const int64_t total = (int64_t)a.tiles * a.groups;
    if (total == 0) return GS_OK;
    a.per_xcd = (int32_t)((total + 7) / 8);
    const int64_t grid = (int64_t)a.per_xcd * 8;
    GS_REQUIRE(grid < 0x7FFFFFFFll, "scoring grid too large (%lld workgroups)", (long long)grid);
    fn<<<(unsigned)grid, waves * 64, lds, s>>>(a);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

template <int WT, int MODE>
int launch_score(ScoreArgs a, int waves, int unroll, hipStream_t s) {
    constexpr size_t acc_bytes = (MODE == kDense64 && WT != GS_W_U8) ? 8 : 4;
    switch (unroll) {
        case 1: return launch_score_u<WT, MODE, 1>(a, waves, acc_bytes, s);
        case 2: return launch_score_u<WT, MODE, 2>(a, waves, acc_bytes, s);
        case 8: return launch_score_u<WT, MODE, 8>(a, waves, acc_bytes, s);
        default: return launch_score_u<WT, MODE, 4>(a, waves, acc_bytes, s);
    }
}

struct SearchPlan {
    int S, cap, rcap, waves, unroll;
    double *margin;
    uint32_t *tau, *cnt, *maxbin, *hist, *cand_doc, *cand_key, *resc_doc, *resc_cnt;
    uint64_t *resc_key;
    void *sample;
};

int check_index(const gs_index *ix) {
    GS_REQUIRE(ix, "null index");
    GS_REQUIRE(ix->wtype >= GS_W_F32 && ix->wtype <= GS_W_U8, "unknown weight type %d", ix->wtype);
    GS_REQUIRE(ix->vocab > 0 && ix->n_docs > 0 && ix->n_docs < 0x7FFFFFFFll, "bad index sizes");
    GS_REQUIRE(ix->tile_log2 >= 8 && ix->tile_log2 <= 13, "tile_log2 %d outside [8, 13]", ix->tile_log2);
    GS_REQUIRE(ix->n_tiles == (int32_t)((ix->n_docs + (1ll << ix->tile_log2) - 1) >> ix->tile_log2),
               "n_tiles %d inconsistent with n_docs and tile_log2", ix->n_tiles);
    GS_REQUIRE(ix->doc_ids_d && ix->weights_d && ix->offsets_d && ix->max_abs_d && ix->dup_d &&
                   ix->tile_bounds_d,
               "index has a null device array");
    return GS_OK;
}

SearchPlan plan_search(const gs_index *ix, int32_t B, int32_t k, const gs_search_opts *o, gs_arena &ar) {
    SearchPlan p;
    p.S = (o && o->sample_tiles > 0) ? o->sample_tiles : kDefaultSample;
    if (p.S > ix->n_tiles) p.S = ix->n_tiles;
    p.cap = (o && o->cand_cap > 0) ? o->cand_cap : kDefaultCandCap;
    if (p.cap < 2 * k) p.cap = 2 * k;
    p.rcap = kRescoreCap;
    p.unroll = (o && o->unroll > 0) ? o->unroll : 4;
    int w = score_waves(ix->tile_log2, 4);
    if (o && (o->waves == 4 || o->waves == 2 || o->waves == 1) && o->waves < w) w = o->waves;
    p.waves = w;
    const int64_t TILE = 1ll << ix->tile_log2;
    p.margin = ar.take<double>(B);
    p.tau = ar.take<uint32_t>(B);
    p.cnt = ar.take<uint32_t>(B);
    p.maxbin = ar.take<uint32_t>(B);
    p.resc_cnt = ar.take<uint32_t>(B);
    p.hist = ar.take<uint32_t>((size_t)B * GS_HIST_BINS);
    p.sample = ar.take<uint32_t>((size_t)B * p.S * TILE);
    p.cand_doc = ar.take<uint32_t>((size_t)B * p.cap);
    p.cand_key = ar.take<uint32_t>((size_t)B * p.cap);
    p.resc_doc = ar.take<uint32_t>((size_t)B * p.rcap);
    p.resc_key = ar.take<uint64_t>((size_t)B * p.rcap);
    return p;
}

ScoreArgs base_args(const gs_index *ix, const int32_t *qt, const void *qw, int32_t T) {
    ScoreArgs a{};
    a.doc = ix->doc_ids_d;
    a.w = ix->weights_d;
    a.offsets = ix->offsets_d;
    a.tb = ix->tile_bounds_d;
    a.qt = qt;
    a.qw = qw;
    a.n_docs = ix->n_docs;
    a.V = ix->vocab;
    a.T = T;
    a.tile_log2 = ix->tile_log2;
    a.n_tiles = ix->n_tiles;
    return a;
}

template <int WT>
int search_impl(const gs_index *ix, const int32_t *qt, const void *qw, int32_t B, int32_t T, int32_t k,
                const gs_search_opts *o, void *out_scores, int64_t *out_ids, int32_t *status, void *ws,
                size_t ws_bytes, hipStream_t s) {
    constexpr bool FP = WT != GS_W_U8;
    gs_arena ar{reinterpret_cast<char *>(ws), 0, ws_bytes};
    SearchPlan p = plan_search(ix, B, k, o, ar);
    if (!ar.ok()) {
        gs_set_error("search workspace too small: need %zu bytes, got %zu", ar.used, ws_bytes);
        return GS_ENOSPC;
    }
    const int64_t TILE = 1ll << ix->tile_log2;
    k_query_prep<WT><<<gs_blocks(B, 256), 256, 0, s>>>(qt, qw, B, T, ix->vocab, ix->max_abs_d, ix->dup_d,
                                                      p.margin, p.tau, p.cnt, p.maxbin);
    k_fill<uint32_t><<<gs_blocks((int64_t)B * GS_HIST_BINS, 256, 4096), 256, 0, s>>>(
        p.hist, (int64_t)B * GS_HIST_BINS, 0u);
    GS_CHECK_LAUNCH();

    // 1. dense sample of tiles [0, S)
    ScoreArgs a = base_args(ix, qt, qw, T);
    a.R = B;
    a.tile_begin = 0;
    a.tiles = p.S;
    a.dense = p.sample;
    a.dense_ld = (int64_t)p.S * TILE;
    a.dense_col0 = 0;
    int rc = launch_score<WT, kDense>(a, p.waves, 4, s);
    if (rc) return rc;
    int64_t sample_cols = (int64_t)p.S * TILE;
    if (sample_cols > ix->n_docs) sample_cols = ix->n_docs;
    k_seed<WT><<<B, 1024, 0, s>>>(p.sample, (int64_t)p.S * TILE, sample_cols, k, p.margin, p.tau, p.cnt, p.maxbin,
                                  p.hist, p.cand_doc, p.cand_key, p.cap);
    GS_CHECK_LAUNCH();

    // 2. fused scoring + emission over the remaining tiles
    if (ix->n_tiles > p.S) {
        ScoreArgs e = base_args(ix, qt, qw, T);
        e.R = B;
        e.tile_begin = p.S;
        e.tiles = ix->n_tiles - p.S;
        e.tau = p.tau;
        e.cnt = p.cnt;
        e.maxbin = p.maxbin;
        e.hist = p.hist;
        e.cand_doc = p.cand_doc;
        e.cand_key = p.cand_key;
        e.margin = p.margin;
        e.cap = p.cap;
        e.k = k;
        if (o && o->ev_score_begin) GS_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(o->ev_score_begin), s));
        rc = launch_score<WT, kEmit>(e, p.waves, p.unroll, s);
        if (rc) return rc;
        if (o && o->ev_score_end) GS_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(o->ev_score_end), s));
    }

    // 3. selection (+ fp64 rescoring for float weights)
    k_select_cands<WT><<<B, kSelThreads, 0, s>>>(p.cand_doc, p.cand_key, p.cnt, p.cap, k, p.margin, p.resc_doc,
                                                 p.resc_cnt, p.rcap, out_scores, out_ids, status);
    GS_CHECK_LAUNCH();
    if (FP) {
        dim3 g((unsigned)((p.rcap + 255) / 256), (unsigned)B);
        k_rescore<WT><<<g, 256, 0, s>>>(ix->doc_ids_d, ix->weights_d, ix->offsets_d, ix->tile_bounds_d, ix->vocab,
                                        ix->n_tiles, ix->tile_log2, qt, reinterpret_cast<const float *>(qw), T,
                                        p.resc_doc, p.resc_cnt, p.rcap, p.resc_key);
        k_select_final<WT><<<B, kSelThreads, 0, s>>>(p.resc_doc, p.resc_key, p.resc_cnt, p.rcap, k, status,
                                                     reinterpret_cast<float *>(out_scores), out_ids);
        GS_CHECK_LAUNCH();
    }
    return GS_OK;
}

template <int WT>
int search_dense_impl(const gs_index *ix, const int32_t *qt, const void *qw, int32_t B, int32_t T, int32_t k,
                      const int32_t *rows, int32_t R, void *out_scores, int64_t *out_ids, void *ws,
                      size_t ws_bytes, hipStream_t s) {
    constexpr size_t acc_bytes = WT == GS_W_U8 ? 4 : 8;
    const int64_t TILE = 1ll << ix->tile_log2;
    const int64_t ld = (int64_t)ix->n_tiles * TILE;
    const int64_t per_row = ld * (int64_t)acc_bytes;
    const int64_t rows_per_pass = (int64_t)(ws_bytes / (size_t)per_row);
    if (rows_per_pass < 1) {
        gs_set_error("dense workspace too small: one row needs %lld bytes, got %zu", (long long)per_row, ws_bytes);
        return GS_ENOSPC;
    }
    const int waves = score_waves(ix->tile_log2, acc_bytes);
    (void)B;
    for (int32_t r0 = 0; r0 < R; r0 += (int32_t)rows_per_pass) {
        const int32_t n = (int32_t)std::min<int64_t>(rows_per_pass, R - r0);
        ScoreArgs a = base_args(ix, qt, qw, T);
        a.rows = rows ? rows + r0 : nullptr;
        a.R = n;
        a.tile_begin = 0;
        a.tiles = ix->n_tiles;
        a.dense = ws;
        a.dense_ld = ld;
        a.dense_col0 = 0;
        // rows == nullptr means queries r0..r0+n-1: shift the query pointers
        if (!rows) {
            a.qt = qt + (int64_t)r0 * T;
            a.qw = reinterpret_cast<const char *>(qw) + (int64_t)r0 * T * (WT == GS_W_U8 ? 1 : 4);
        }
        int rc = launch_score<WT, kDense64>(a, waves, 4, s);
        if (rc) return rc;
        k_select_dense<WT><<<n, kSelThreads, 0, s>>>(ws, ld, ix->n_docs, k, rows, r0, out_scores, out_ids);
        GS_CHECK_LAUNCH();
    }
    return GS_OK;
}

}  // namespace

// ====================================================================== C ABI

extern "C" int gs_search_workspace(const gs_index *index, int32_t B, int32_t T, int32_t k,
                                   const gs_search_opts *opts, size_t *bytes) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(B > 0 && T > 0 && k > 0 && bytes, "bad search sizes");
    gs_arena ar{nullptr, 0, 0};
    plan_search(index, B, k, opts, ar);
    *bytes = ar.used + 256;
    return GS_OK;
}

extern "C" int gs_search(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B,
                         int32_t T, int32_t k, const gs_search_opts *opts, void *out_scores_d, int64_t *out_ids_d,
                         int32_t *status_d, void *workspace_d, size_t workspace_bytes, void *stream) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(B > 0 && T > 0, "empty query batch (B=%d, T=%d)", B, T);
    GS_REQUIRE(k >= 1 && k <= kMaxK && (int64_t)k <= index->n_docs, "k=%d outside [1, min(n_docs, %d)]", k, kMaxK);
    GS_REQUIRE(q_terms_d && q_weights_d && out_scores_d && out_ids_d && status_d && workspace_d, "null pointer");
    hipStream_t s = gs_stream(stream);
    switch (index->wtype) {
        case GS_W_F32:
            return search_impl<GS_W_F32>(index, q_terms_d, q_weights_d, B, T, k, opts, out_scores_d, out_ids_d,
                                         status_d, workspace_d, workspace_bytes, s);
        case GS_W_F16:
            return search_impl<GS_W_F16>(index, q_terms_d, q_weights_d, B, T, k, opts, out_scores_d, out_ids_d,
                                         status_d, workspace_d, workspace_bytes, s);
        default:
            return search_impl<GS_W_U8>(index, q_terms_d, q_weights_d, B, T, k, opts, out_scores_d, out_ids_d,
                                        status_d, workspace_d, workspace_bytes, s);
    }
}

extern "C" int gs_search_dense_workspace(const gs_index *index, int32_t rows_per_pass, size_t *bytes) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(rows_per_pass > 0 && bytes, "bad arguments");
    const size_t acc = index->wtype == GS_W_U8 ? 4 : 8;
    *bytes = (size_t)rows_per_pass * (size_t)index->n_tiles * ((size_t)1 << index->tile_log2) * acc;
    return GS_OK;
}

extern "C" int gs_search_dense(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B,
                               int32_t T, int32_t k, const int32_t *rows_d, int32_t R, void *out_scores_d,
                               int64_t *out_ids_d, void *workspace_d, size_t workspace_bytes, void *stream) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(B > 0 && T > 0 && R >= 0 && R <= B, "bad sizes (B=%d, T=%d, R=%d)", B, T, R);
    GS_REQUIRE(k >= 1 && k <= kMaxK && (int64_t)k <= index->n_docs, "k=%d outside [1, min(n_docs, %d)]", k, kMaxK);
    GS_REQUIRE(q_terms_d && q_weights_d && out_scores_d && out_ids_d && workspace_d, "null pointer");
    if (R == 0) return GS_OK;
    hipStream_t s = gs_stream(stream);
    switch (index->wtype) {
        case GS_W_F32:
            return search_dense_impl<GS_W_F32>(index, q_terms_d, q_weights_d, B, T, k, rows_d, R, out_scores_d,
                                               out_ids_d, workspace_d, workspace_bytes, s);
        case GS_W_F16:
            return search_dense_impl<GS_W_F16>(index, q_terms_d, q_weights_d, B, T, k, rows_d, R, out_scores_d,
                                               out_ids_d, workspace_d, workspace_bytes, s);
        default:
            return search_dense_impl<GS_W_U8>(index, q_terms_d, q_weights_d, B, T, k, rows_d, R, out_scores_d,
                                              out_ids_d, workspace_d, workspace_bytes, s);
    }
}

extern "C" size_t gs_compacted_topk_workspace(int32_t B, int32_t max_cand) {
    gs_arena ar{nullptr, 0, 0};
    ar.take<int32_t>((size_t)B * max_cand);
    ar.take<float>((size_t)B * max_cand);
    return ar.used + 256;
}

extern "C" int gs_compacted_topk(const float *scores_d, int64_t ld, int32_t B, int64_t L, const float *tau_d,
                                 int32_t k, int32_t max_cand, float *out_values_d, int64_t *out_idx_d,
                                 int32_t *counts_d, void *workspace_d, size_t workspace_bytes, void *stream) {
    GS_REQUIRE(B > 0 && L > 0 && ld >= L, "bad shape (B=%d, L=%lld, ld=%lld)", B, (long long)L, (long long)ld);
    GS_REQUIRE(L < 0x7FFFFFFFll, "row length %lld exceeds int32", (long long)L);
    GS_REQUIRE(k >= 1 && k <= kMaxK && (int64_t)k <= L, "k=%d outside [1, min(L, %d)]", k, kMaxK);
    GS_REQUIRE(max_cand >= k, "max_cand %d < k %d", max_cand, k);
    GS_REQUIRE(scores_d && out_values_d && out_idx_d && counts_d, "null pointer");
    hipStream_t s = gs_stream(stream);
    gs_arena ar{reinterpret_cast<char *>(workspace_d), 0, workspace_bytes};
    int32_t *cidx = ar.take<int32_t>((size_t)B * max_cand);
    float *cval = ar.take<float>((size_t)B * max_cand);
    if (!ar.ok() || !workspace_d) {
        gs_set_error("compacted_topk workspace too small: need %zu bytes, got %zu", ar.used, workspace_bytes);
        return GS_ENOSPC;
    }
    k_fill<int32_t><<<gs_blocks(B, 256), 256, 0, s>>>(counts_d, B, 0);
    if (tau_d) {
        dim3 g(gs_blocks(L, 256, 4096), (unsigned)B);
        k_compact<<<g, 256, 0, s>>>(scores_d, ld, L, tau_d, cidx, cval, counts_d, max_cand);
    } else {
        k_fill<int32_t><<<gs_blocks(B, 256), 256, 0, s>>>(counts_d, B, (int32_t)L);
    }
    GS_CHECK_LAUNCH();
    k_select_compacted<<<B, kSelThreads, 0, s>>>(scores_d, ld, L, tau_d, cidx, cval, tau_d ? counts_d : nullptr,
                                                 max_cand, k, out_values_d, out_idx_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_scatter_add(const gs_index *index, const int64_t *lo_d, const int64_t *hi_d,
                              const int32_t *q_terms_d, const void *q_weights_d, int32_t B, int32_t T, void *out_d,
                              int64_t chunk_start, int64_t chunk_len, int64_t out_stride, int32_t block_pl,
                              void *stream) {
    GS_REQUIRE(index && index->doc_ids_d && index->weights_d && index->offsets_d && index->lengths_d,
               "index has a null device array");
    GS_REQUIRE(B > 0 && T > 0 && chunk_len >= 0 && out_stride >= chunk_len, "bad sizes");
    GS_REQUIRE(block_pl > 0 && (block_pl & (block_pl - 1)) == 0, "block_pl must be a positive power of 2, got %d",
               block_pl);
    GS_REQUIRE((lo_d == nullptr) == (hi_d == nullptr), "lo and hi must both be given or both be NULL");
    GS_REQUIRE((int64_t)B * T < 0x7FFFFFFFll, "too many (query, term) programs");
    hipStream_t s = gs_stream(stream);
    // (query, term) programs, each split over `parts` workgroups of 256 lanes
    int parts = block_pl >= 256 ? block_pl / 256 : 1;
    if (parts > 64) parts = 64;
    dim3 g((unsigned)(B * T), (unsigned)parts);
    switch (index->wtype) {
        case GS_W_F32:
            k_scatter_atomic<GS_W_F32><<<g, 256, 0, s>>>(index->doc_ids_d, index->weights_d, index->offsets_d,
                                                         index->lengths_d, lo_d, hi_d, q_terms_d, q_weights_d, T,
                                                         index->vocab, out_d, chunk_start, chunk_len, out_stride);
            break;
        case GS_W_F16:
            k_scatter_atomic<GS_W_F16><<<g, 256, 0, s>>>(index->doc_ids_d, index->weights_d, index->offsets_d,
                                                         index->lengths_d, lo_d, hi_d, q_terms_d, q_weights_d, T,
                                                         index->vocab, out_d, chunk_start, chunk_len, out_stride);
            break;
        default:
            k_scatter_atomic<GS_W_U8><<<g, 256, 0, s>>>(index->doc_ids_d, index->weights_d, index->offsets_d,
                                                        index->lengths_d, lo_d, hi_d, q_terms_d, q_weights_d, T,
                                                        index->vocab, out_d, chunk_start, chunk_len, out_stride);
    }
    GS_CHECK_LAUNCH();
    return GS_OK;
}
