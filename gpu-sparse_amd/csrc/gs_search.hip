// Exact batched SPLADE scoring and top-k selection for gfx950.
//
// What is computed is the reference's scatter-add (src/triton_kernel.py:93-156):
//     score[q, d] = sum over valid terms j of q_w[q, j] * w(q_t[q, j], d)
// followed by an exact top-k (torch.topk at triton_kernel.py:199, or the
// chunked / threshold-compacted selection of src/fused_topk.py:106-160).
//
// How it is computed here:
//  * Documents are cut into tiles of 2^tile_log2 docs and queries into groups of
//    G.  One workgroup owns one (tile, group) pair and keeps the G queries'
//    scores for that tile in LDS.  It walks the union of the group's terms,
//    reads each posting inside the tile once (per-(term, tile) bounds) and adds
//    its contribution to every query of the group holding that term.  No
//    [B, N] accumulator exists and no global atomics are issued for scores.
//  * LDS accumulation is integer: on gfx950 ds_add_u32 sustains ~17x the rate
//    of ds_add_f32.  Float configurations add per-query fixed-point values
//    rint(q * w * 2^e), with 2^e chosen so the sum of |contributions| stays
//    below 2^31; uint8 configurations add the exact uint32 products.
//  * Workgroups are mapped tile-major and XCD-aware, so the workgroups resident
//    on one XCD share a tile's posting lines in that XCD's L2.
//  * Selection is fused into the scoring kernel.  A dense sample of the first
//    tiles seeds a per-query lower bound tau on the k-th (fixed-point) score;
//    every workgroup then emits only docs scoring >= tau - margin (ballot
//    compaction, one atomic per 64 docs), counts them in a per-query histogram
//    of score bins and raises tau from that histogram.  tau never exceeds the
//    true k-th fixed-point score, so no doc of the answer is dropped.
//  * Float configurations then take the fixed-point k-th score tau' and a
//    rigorous rounding bound E: every doc whose fp64 score can reach the top k
//    has fixed >= tau' - 2E; those are rescored in fp64 in query-term order
//    (exactly the fp64 scatter-add) and ordered (score desc, doc asc).  uint8
//    configurations are exact as accumulated.
//  * A row whose candidates overflow, or whose k-th score is not clear of zero
//    by the margin, is flagged and finished by the dense path (fp64 / uint32
//    tiles written to a full row, then an exact radix select).
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "gs_topk.h"

namespace {

using namespace gs;

constexpr int kRescoreCap = 16384;   // candidates rescored per query before the dense fallback
constexpr int kHeadShift = 20;       // bits of the heavy-term sums dropped in their coarse copy (12 bits left)
constexpr int kHeadBlock = GS_HEAD_BLOCK;  // docs per workgroup of k_head_scores
constexpr int kHscRow = kHeadBlock * 3 / 2;  // bytes of one (doc block, slot) row of 12-bit coarse sums
typedef uint32_t gs_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t gs_u32x2 __attribute__((ext_vector_type(2)));
constexpr int64_t kSeedMinDocs = 4096;    // fewest docs of the default first tiles scored with tau = 0
constexpr int64_t kSeedDocs = 32768;      // most docs of the default first tiles scored with tau = 0
constexpr int kDefaultCandCap = 65536;      // fewest candidate slots per query of the default cap
constexpr int64_t kCandBudget = 1ll << 24;  // candidate slots of a batch that the default cap spreads over it
constexpr int kMaxCandCap = 1 << 22;        // most candidate slots per query of the default cap
constexpr int64_t kSeedFillWgs = 256;       // workgroups (tiles x query groups) a default seed launch aims at
constexpr int64_t kSeedMaxTiles = 64;       // most tiles of a default seed widened towards that
constexpr int64_t kPairMinWgs = 12288;    // workgroups (~48 per CU) needed before a workgroup scores two tiles
constexpr int64_t kTripleMinWgs = 49152;  // and before it scores three
constexpr size_t kTileLds = 144 * 1024;  // LDS of the fp64 / uint32 row tiles of one dense-path workgroup
// LDS of the score slices of one fused-scoring workgroup (2 queries x 8192 docs):
// two such workgroups share a CU, so one's set-up and emission (latency-bound)
// overlap the other's adds
constexpr size_t kUnionTileLds = 64 * 1024;
constexpr int kGroupSortCap = 8192;      // term entries of one query group sorted in LDS
static_assert(kGroupSortCap < (1 << 15), "union terms pack (entry count << 16 | first entry) into int32");
// dynamic-LDS cap requested per kernel: 160 KiB per workgroup minus room for static LDS
constexpr size_t kLdsPerWg = 160 * 1024;     // gfx950 LDS of one workgroup (static + dynamic)
constexpr size_t kStaticLdsBudget = 6144;    // static LDS allowed next to the largest dynamic request

// Lets `fn` take all the LDS of a workgroup: 160 KiB minus its static LDS.
inline hipError_t allow_full_lds(const void *fn) {
    hipFuncAttributes at;
    const hipError_t e = hipFuncGetAttributes(&at, fn);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kLdsPerWg - at.sharedSizeBytes));
}


template <class T>
__global__ void k_fill(T *p, int64_t n, T v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// ---------------------------------------------------------------------- per-query prep

// Fixed-point scale and selection margin of each query.  A doc's score is a sum
// of at most n = sum_j (1 + dup[t_j]) products, and sum |products| <= M =
// sum_j |q_j| * max|w(t_j)| * (1 + dup[t_j]).  With scale S = 2^e,
// c = trunc(fl32(q * w) * S) is within 2^-24 |q w| S + 1 of q w S, so
//   |sum c / S - exact| <= E = 2^-24 M + n / S,   |sum c| <= M S (1 + 2^-24),
// and e is the largest exponent keeping the latter below 2^31.  The fp64
// rescoring is within g64(2n) M of exact.  Any doc of the fp64 top k then has a
// fixed-point score >= tau' - 2 (E + g64 M) S, which is the margin `mfix`.
// uint8 impacts: S = 1, exact, margin 0.
//
// With the packed copy (pk != 0) of float weights, the products are integers
// qi * wq with wq = rint(w 2^s) (s = pk_shift, |wq| <= W_t = rint(max|w(t)| 2^s))
// and qi = rint(q 2^f); `scale` then holds 2^f and the fixed-point scale is
// S = 2^(f+s).  Per product |qi wq - q w S| <= |qi - q 2^f| |wq| + |q| 2^f |wq -
// w 2^s| <= W_t / 2 + |q| 2^f / 2, so with Bw = sum_j W_j (1 + dup) and Q = sum_j
// |q_j| (1 + dup):  |sum - exact S| <= Bw / 2 + Q 2^f / 2.  f is the largest
// exponent with sum |qi wq| <= A 2^f + Bw / 2 < 2^31 (A = sum_j |q_j| W_j (1 +
// dup)) and |qi| < 2^23 (the operand width of v_mul_i32_i24).  A term with W_t >
// 32767 (a copy packed with too large a shift), or no feasible f, gets the
// margin 2^31 - 1: the row is then finished by the dense path.
template <int WT>
__global__ void k_query_prep(const int32_t *__restrict__ qt, const void *__restrict__ qw, int32_t B, int32_t T,
                             int32_t V, const float *__restrict__ max_abs, const int32_t *__restrict__ dup,
                             int32_t pk, int32_t pk_shift, float *__restrict__ scale, uint32_t *__restrict__ mfix,
                             uint32_t *__restrict__ tau, uint32_t *__restrict__ cnt, uint32_t *__restrict__ maxbin) {
    // one wave per query; the lanes sum over its terms
    const int q = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6);
    const int lane = gs_lane();
    if (q >= B) return;
    if (lane == 0) {
        tau[q] = 0;
        cnt[q] = 0;
        maxbin[q] = 0;
    }
    if (WT == GS_W_U8) {
        if (lane == 0) {
            scale[q] = 1.0f;
            mfix[q] = 0;
        }
        return;
    }
    // M and n as fp64 sums in any order: the factor (1 + 1e-12) below covers the
    // rounding of a sum of up to 8192 non-negative terms
    double M = 0.0, n = 0.0, A = 0.0, Bw = 0.0, Q = 0.0, qmax = 0.0, Wmax = 0.0;
    for (int j = lane; j < T; j += 64) {
        const int32_t t = qt[(int64_t)q * T + j];
        if ((uint32_t)t >= (uint32_t)V) continue;
        const double m = 1.0 + (double)dup[t];
        const double aq = fabs((double)reinterpret_cast<const float *>(qw)[(int64_t)q * T + j]);
        M += aq * (double)max_abs[t] * m;
        n += m;
        if (pk) {
            const double W = rint(ldexp((double)max_abs[t], pk_shift));
            A += aq * W * m;
            Bw += W * m;
            Q += aq * m;
            qmax = fmax(qmax, aq);
            Wmax = fmax(Wmax, W);
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        M += __shfl_xor(M, d, 64);
        n += __shfl_xor(n, d, 64);
        A += __shfl_xor(A, d, 64);
        Bw += __shfl_xor(Bw, d, 64);
        Q += __shfl_xor(Q, d, 64);
        qmax = fmax(qmax, __shfl_xor(qmax, d, 64));
        Wmax = fmax(Wmax, __shfl_xor(Wmax, d, 64));
    }
    if (lane != 0) return;
    M *= 1.0 + 1e-12;  // fp64 rounding of the sum itself
    const double g64 = (2.0 * n + 2.0) * 0x1p-53 / (1.0 - (2.0 * n + 2.0) * 0x1p-53);
    if (pk) {
        A *= 1.0 + 1e-12;
        Bw *= 1.0 + 1e-12;
        Q *= 1.0 + 1e-12;
        const double room = 2147483646.0 - 0.5 * Bw;
        int f = 100;
        if (A > 0.0) f = (int)floor(log2(room / A));
        if (qmax > 0.0) f = min(f, (int)floor(log2(8388607.0 / qmax)));
        f = f > 100 ? 100 : (f < -100 ? -100 : f);
        // the floors above are in fp64; step down while a bound is not met exactly
        while (f > -100 && (A * ldexp(1.0, f) >= room || qmax * ldexp(1.0, f) + 0.5 >= 8388608.0)) --f;
        const bool ok = room > 0.0 && Wmax <= 32767.0 && A * ldexp(1.0, f) < room &&
                        qmax * ldexp(1.0, f) + 0.5 < 8388608.0;
        const double Ef = 0.5 * Bw + 0.5 * Q * ldexp(1.0, f);  // fixed-point units
        double mf = ceil(2.0 * (Ef * (1.0 + 1e-9) + g64 * M * ldexp(1.0, f + pk_shift))) + 2.0;
        if (!ok || mf > 2147483647.0) mf = 2147483647.0;
        scale[q] = (float)ldexp(1.0, f);
        mfix[q] = (uint32_t)mf;
        return;
    }
    int e = 30;
    if (M > 0.0) {
        const double lim = (2147483647.0 - n - 2.0) / (M * (1.0 + 0x1p-23));
        e = (int)floor(log2(lim));
        e = e > 100 ? 100 : (e < -100 ? -100 : e);
    }
    const double S = ldexp(1.0, e);
    const double E = 0x1p-24 * M * (1.0 + 1e-9) + n / S + g64 * M;
    double mf = ceil(2.0 * E * S) + 2.0;
    if (mf > 2147483647.0) mf = 2147483647.0;
    scale[q] = (float)S;
    mfix[q] = (uint32_t)mf;
}

// Lower bound on (positive) integer scores whose fp32 image lies in bins >= b.
__device__ __forceinline__ uint32_t int_threshold_of_bin(uint32_t b) {
    const double e = (double)gs_bin_edge(b);
    return (uint32_t)floor(e / (1.0 + 0x1p-23));
}

// Candidate threshold: tau lowered by the margin, at least 1 (only positive scores qualify).
__device__ __forceinline__ uint32_t emit_threshold(uint32_t tau, uint32_t mfix) {
    return tau > mfix + 1u ? tau - mfix : 1u;
}

// Recompute tau[q] from the histogram (bins <= top scanned downward): the lower
// edge of the highest bin b with count(bins >= b) >= k.  Whole wave calls it.
__device__ void raise_tau(uint32_t *tau, const uint32_t *hist, uint32_t top, int k) {
    const int lane = gs_lane();
    const uint32_t cur = gs_load_relaxed(tau);
    const uint32_t cur_bin = gs_bin_of((float)cur);
    uint32_t cum = 0;
    for (int b = (int)top; b >= 0 && b + 1 > (int)cur_bin; b -= 64) {
        const int bb = b - lane;
        const uint32_t c = bb >= 0 ? gs_load_relaxed(hist + bb) : 0u;
        const uint32_t inc = gs_wave_incl_scan(c);
        const uint64_t hit = __ballot(cum + inc >= (uint32_t)k);
        if (hit) {
            const int l = __ffsll((unsigned long long)hit) - 1;
            const uint32_t bin = (uint32_t)(b - l);
            if (lane == 0 && bin > cur_bin) atomicMax(tau, int_threshold_of_bin(bin));
            return;
        }
        cum += __shfl(inc, 63, 64);
    }
}

template <class A>
__device__ __forceinline__ void lds_add(A *p, A v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Fixed-point contribution of one posting: trunc(fl32(qs * w)) with qs = q * 2^e
// (one multiply and one v_cvt_i32_f32); uint8: the exact product (both factors
// < 2^8, one full-rate v_mul_u32_u24).
template <int WT>
__device__ __forceinline__ uint32_t fixed_contrib(uint32_t qbits, typename gs_weight<WT>::store_t w) {
    if (WT == GS_W_U8) return __umul24(qbits, (uint32_t)w);
    return (uint32_t)(int32_t)(__uint_as_float(qbits) * (float)gs_weight<WT>::decode(w));
}

// Contribution of one packed posting word (offset in bits 0-15, weight above):
// uint8 weight times the uint8 query weight, or int16 rint(w 2^s) times the
// integer query weight rint(q 2^f) (|.| < 2^23); exact 32-bit products either way
// (v_mul_{u32_u24,i32_i24} reading the weight half-word through SDWA).
template <int WT>
__device__ __forceinline__ uint32_t packed_contrib(uint32_t qv, uint32_t word) {
    if (WT == GS_W_U8) return __umul24(qv, (word >> 16) & 0xFFu);
    return (uint32_t)__mul24((int32_t)qv, (int32_t)word >> 16);
}

// ---------------------------------------------------------------------- dense per-query tiles

struct DenseArgs {
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
    void *dense;
    int64_t dense_ld, dense_col0;
};

// One wave owns one (query, tile): it walks the query's terms in order, adds
// every posting of the tile into its LDS slice and writes the slice to a dense
// row: fp64 for float weights (terms added in query order, i.e. the fp64
// scatter-add itself) or uint32 for uint8 impacts -- the exact dense path.
template <int WT, int UNROLL>
__global__ void __launch_bounds__(512) k_score_dense(const DenseArgs a) {
    using W = gs_weight<WT>;
    using store_t = typename W::store_t;
    constexpr bool kF64 = WT != GS_W_U8;
    using acc_t = typename std::conditional<kF64, double, uint32_t>::type;

    extern __shared__ __align__(16) unsigned char lds_raw[];
    const int waves = (int)(blockDim.x >> 6);
    const int wave = gs_uniform((int)(threadIdx.x >> 6));
    const int lane = gs_lane();

    // XCD-aware block order: workgroup i runs on XCD i % 8; each XCD gets a
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
        uint32_t qbits = 0;
        double wq64 = 0.0;
        if (WT == GS_W_U8)
            qbits = reinterpret_cast<const uint8_t *>(a.qw)[(int64_t)q * a.T + j];
        else
            wq64 = (double)reinterpret_cast<const float *>(a.qw)[(int64_t)q * a.T + j];
        auto contrib = [&](store_t wv) -> acc_t {
            if (kF64) return (acc_t)(wq64 * (double)W::decode(wv));
            return (acc_t)fixed_contrib<WT>(qbits, wv);
        };
        int p = lo + lane;
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
    acc_t *out = reinterpret_cast<acc_t *>(a.dense) + (int64_t)r * a.dense_ld + (doc0 - a.dense_col0);
    for (int i = lane; i < ncols; i += 64) out[i] = acc[i];
}

// ---------------------------------------------------------------------- query-group unions

// Queries are processed in groups of G.  Per group, the (term, query slot,
// weight) entries of its valid query terms are sorted by (term, slot, position)
// so that each distinct term owns a contiguous entry range; u_term / u_ebeg list
// the distinct terms (see the reordering at the end) with u_ebeg = entry count
// << 16 | first entry.  Entry weights are stored pre-scaled: q * 2^e_q as fp32
// bits for float weights, or with the packed copy (pk != 0) the integer rint(q *
// 2^f) (k_query_prep), and the uint8 weight for impacts.  With `hrank` (the
// hybrid scorer) the heavy terms are left out: the unions hold the tail terms.
template <int WT>
__global__ void __launch_bounds__(1024)
    k_group_terms(const int32_t *__restrict__ qt, const void *__restrict__ qw, const float *__restrict__ scale,
                  int32_t pk, int32_t B, int32_t T, int32_t V, int32_t G, int32_t ecap,
                  const int16_t *__restrict__ hrank, int32_t *__restrict__ u_term, int32_t *__restrict__ u_ebeg,
                  int32_t *__restrict__ u_count, uint2 *__restrict__ e_sw) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    __shared__ int32_t s_sh[17];
    __shared__ int32_t s_tot;
    const int grp = blockIdx.x;
    const int nq = min(G, B - grp * G);
    const int n = nq * T;
    int np = 1;
    while (np < n) np <<= 1;
    uint64_t *key = reinterpret_cast<uint64_t *>(lds_raw);
    uint32_t *wv = reinterpret_cast<uint32_t *>(key + np);
    for (int i = threadIdx.x; i < np; i += blockDim.x) {
        uint64_t kk = ~0ull;
        uint32_t w = 0;
        if (i < n) {
            const int g = i / T, j = i % T;
            const int q = grp * G + g;
            const int64_t src = (int64_t)q * T + j;
            const int32_t t = qt[src];
            if ((uint32_t)t < (uint32_t)V && !(hrank && hrank[t] >= 0)) {
                kk = ((uint64_t)(uint32_t)t << 32) | ((uint64_t)g << 20) | (uint64_t)j;
                if (WT == GS_W_U8) {
                    w = (uint32_t) reinterpret_cast<const uint8_t *>(qw)[src];
                } else {
                    const float x = reinterpret_cast<const float *>(qw)[src] * scale[q];  // exact: scale = 2^f
                    w = pk ? (uint32_t)(int32_t)rintf(x) : __float_as_uint(x);
                }
            }
        }
        key[i] = kk;
        wv[i] = w;
    }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t ka = key[lo], kb = key[hi];
                if ((ka > kb) == up) {
                    key[lo] = kb;
                    key[hi] = ka;
                    const uint32_t t = wv[lo];
                    wv[lo] = wv[hi];
                    wv[hi] = t;
                }
            }
            __syncthreads();
        }
    }
    // a term starts where its id differs from the previous entry's
    int carry = 0;
    for (int base = 0; base < np; base += blockDim.x) {
        const int i = base + threadIdx.x;
        const uint64_t kk = i < np ? key[i] : ~0ull;
        const bool valid = kk != ~0ull;
        const bool head = valid && (i == 0 || (key[i - 1] >> 32) != (kk >> 32));
        const int v = head;
        int x = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(x, d, 64);
            if (gs_lane() >= d) x += o;
        }
        if (gs_lane() == 63) s_sh[threadIdx.x >> 6] = x;
        __syncthreads();
        if (threadIdx.x == 0) {
            int acc = 0;
            for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
                const int s = s_sh[w];
                s_sh[w] = acc;
                acc += s;
            }
            s_sh[16] = acc;
        }
        __syncthreads();
        const int ex = carry + s_sh[threadIdx.x >> 6] + x - v;
        const int tot = s_sh[16];
        __syncthreads();
        if (valid) {
            e_sw[(int64_t)grp * ecap + i] = make_uint2((uint32_t)((kk >> 20) & 0xFFFu), wv[i]);
            if (head) {
                u_term[(int64_t)grp * ecap + ex] = (int32_t)(kk >> 32);
                u_ebeg[(int64_t)grp * (ecap + 1) + ex] = i;
            }
        }
        carry += tot;
    }
    if (threadIdx.x == 0) s_tot = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < np; i += blockDim.x)
        if (key[i] != ~0ull && (i + 1 == np || key[i + 1] == ~0ull)) s_tot = i + 1;
    __syncthreads();
    if (threadIdx.x == 0) {
        u_count[grp] = carry;
        u_ebeg[(int64_t)grp * (ecap + 1) + carry] = s_tot;
    }
    __syncthreads();
    // Reorder the union terms by entry count, descending (ties by term id), and
    // store each as (count << 16 | first entry).  The scorer hands chunks to its
    // waves round-robin in this order, so the last chunks of a tile are the
    // cheapest ones and the waves reach the closing barrier close together.
    int32_t *ut = u_term + (int64_t)grp * ecap;
    int32_t *ue = u_ebeg + (int64_t)grp * (ecap + 1);
    const int U = carry;
    for (int i = threadIdx.x; i < np; i += blockDim.x)
        key[i] = i < U ? ((uint64_t)(uint32_t)(kGroupSortCap - (ue[i + 1] - ue[i])) << 32) | (uint32_t)i : ~0ull;
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t ka = key[lo], kb = key[hi];
                if ((ka > kb) == up) {
                    key[lo] = kb;
                    key[hi] = ka;
                }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < U; i += blockDim.x) {
        const int u = (int)(uint32_t)key[i];
        const int m = kGroupSortCap - (int)(key[i] >> 32);
        key[i] = ((uint64_t)(uint32_t)ut[u] << 32) | (uint32_t)((m << 16) | ue[u]);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < U; i += blockDim.x) {
        ut[i] = (int32_t)(key[i] >> 32);
        ue[i] = (int32_t)(uint32_t)key[i];
    }
}

// ---------------------------------------------------------------------- query grouping

// Each posting is loaded once per (doc tile, query group) and added to every slot
// of the group holding its term, so groups whose queries share long lists load
// fewer postings.  A query's signature is the set of the index's kSignTerms (64)
// most frequent terms it holds: a 64-bit mask, bit 63 = the most frequent term.  Per
// block of NB = G floor(1024 / G) queries: masks from all (query, term) entries
// at once (LDS atomic or), then the queries sorted by mask (descending, then
// query index), so that queries holding the same most frequent terms become
// neighbours and share groups.  perm[slot] = query.  The order only moves
// queries between groups: every query's result is the same in any order.
__global__ void __launch_bounds__(1024)
    k_group_order(const int32_t *__restrict__ qt, int32_t B, int32_t T, int32_t V, const int32_t *__restrict__ heavy,
                  int32_t G, int32_t *__restrict__ perm) {
    __shared__ int32_t h_term[256];  // open-addressing table: heavy term -> mask bit
    __shared__ int32_t h_bit[256];
    __shared__ uint64_t s_mask[1024];
    __shared__ uint32_t s_idx[1024];
    const int tid = threadIdx.x;
    const int NB = G * (1024 / G);
    const int base = blockIdx.x * NB;
    const int n = min(NB, B - base);
    int np = 1;
    while (np < n) np <<= 1;
    if (tid < 256) h_term[tid] = -1;
    s_mask[tid] = 0;
    s_idx[tid] = (uint32_t)tid;  // entries past n sort last: mask 0, larger index
    __syncthreads();
    if (tid < kSignTerms) {
        const int32_t t = heavy[tid];
        if (t >= 0) {
            uint32_t h = ((uint32_t)t * 2654435761u) >> 24;
            while (atomicCAS(&h_term[h], -1, t) != -1) h = (h + 1) & 255u;
            h_bit[h] = 63 - tid;
        }
    }
    __syncthreads();
    // masks from the block's (query, term) entries: each thread loads 8 entries
    // at a time (coalesced, all in flight together), then looks them up
    const int ne = n * T;
    const int32_t *rows = qt + (int64_t)base * T;
    for (int e0 = 0; e0 < ne; e0 += 8 * 1024) {
        int32_t tv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int e = e0 + r * 1024 + tid;
            tv[r] = e < ne ? rows[e] : -1;
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int32_t t = tv[r];
            if ((uint32_t)t >= (uint32_t)V) continue;
            uint32_t h = ((uint32_t)t * 2654435761u) >> 24;
            int32_t x;
            while ((x = h_term[h]) != t && x >= 0) h = (h + 1) & 255u;
            if (x == t)
                __hip_atomic_fetch_or(&s_mask[(uint32_t)(e0 + r * 1024 + tid) / (uint32_t)T], 1ull << h_bit[h],
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            const int j = tid ^ stride;
            if (tid < np && j > tid) {
                const uint64_t mi = s_mask[tid], mj = s_mask[j];
                const uint32_t ii = s_idx[tid], ij = s_idx[j];
                const bool j_first = mj > mi || (mj == mi && ij < ii);
                if (j_first == ((tid & size) == 0)) {
                    s_mask[tid] = mj;
                    s_mask[j] = mi;
                    s_idx[tid] = ij;
                    s_idx[j] = ii;
                }
            }
        }
    __syncthreads();
    if (tid < n) perm[base + tid] = base + (int)s_idx[tid];
}

// qt_p / qw_p rows in slot order: row s is query perm[s]
template <int WT>
__global__ void k_permute_queries(const int32_t *__restrict__ qt, const void *__restrict__ qw,
                                  const int32_t *__restrict__ perm, int32_t B, int32_t T, int32_t *__restrict__ qt_p,
                                  void *__restrict__ qw_p) {
    using qw_t = typename gs_weight<WT>::qw_t;
    const int64_t n = (int64_t)B * T;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t src = (int64_t)perm[i / T] * T + i % T;
        qt_p[i] = qt[src];
        reinterpret_cast<qw_t *>(qw_p)[i] = reinterpret_cast<const qw_t *>(qw)[src];
    }
}

// ---------------------------------------------------------------------- group-tile scoring

struct UnionArgs {
    const int32_t *doc;
    const void *w;
    const void *pk;  // packed scoring copy for this tile size, or null
    const int64_t *offsets;
    const int32_t *tb;  // [V][n_tiles + 1]
    int64_t n_docs;
    int32_t V, tile_log2, n_tiles;
    int32_t B, G, n_groups, ecap;
    const int32_t *u_term, *u_ebeg, *u_count;
    const uint2 *e_sw;  // (query slot, scaled query weight) per entry
    int32_t tile_begin, tiles, tiles_per_wg, per_xcd;
    uint32_t *tau, *cnt, *maxbin, *hist, *cand_doc, *cand_key;
    const uint32_t *mfix;
    int32_t cap, k;
    int32_t local_k;  // > 0: threshold each slot at its tile's local k-th score too (seed launch)
    const uint8_t *hsc;  // HD: 12-bit coarse heavy-term sums, block-major rows (k_head_scores), the slices' start
    int64_t hsc_ld;      // slots per 512-doc block of hsc
};

constexpr int kUnionThreads = 512;  // 8 waves; two workgroups per CU
constexpr int kUnionBatch = 220;    // union terms described in LDS at a time
constexpr int kEmitChunks = (int)(kUnionTileLds / 4 / 256);  // 256-doc emission chunks of one workgroup
constexpr int kLocalBins = 256;  // bins of the per-slot score histogram of the seed launch
constexpr int kLocalSlots = 4;   // slots per workgroup that get a local threshold
constexpr int kEmitReads = 4;    // emission chunks a wave reads at once in the counting pass

// LDS bytes of k_score_union besides the G score slices
constexpr size_t kUnionMetaLds =
    (size_t)kUnionBatch * 8 + (size_t)kUnionBatch * 4 + (size_t)(kUnionBatch + 2) * 8 + (size_t)kUnionBatch * 12;
static_assert(kUnionTileLds + kUnionMetaLds + kStaticLdsBudget <= kLdsPerWg / 2,
              "two scoring workgroups must fit the 160 KiB of LDS of a CU");

// ---------------------------------------------------------------------- candidate emission

struct EmitArgs {
    uint32_t *tau, *cnt, *maxbin, *hist, *cand_doc, *cand_key;
    int32_t G, cap, k;
};

// Emission of one tile's slices (G int32 slices of 1 << (cps_log2 + 8) docs at
// LDS word `acc`, slot g's slice at word g << (cps_log2 + 8)): every doc at or
// above its slot's threshold s_thr[g] (set and fenced by the caller) becomes a
// candidate (doc, key) of query grp * G + g, counted in that query's histogram,
// and tau is raised from the histogram as the counts grow.  The slices are
// scanned in 256-doc chunks, 4 docs per lane (one 16-byte LDS read); slices are
// zero or hold sums of every doc of the tile (docs past n_docs add nothing), and
// thresholds >= 1 make the signed compare also reject zero and negative sums.
// Pass 1 counts each chunk's candidates; one wave per slot scans the slot's
// chunk counts (one per lane) and reserves the slot's range with one global
// atomic; pass 2 revisits only the chunks holding candidates (a wave reads its
// chunk counts at once, one per lane).  Whole workgroup (kUnionThreads) calls it.
__device__ __forceinline__ void emit_slices(const EmitArgs &a, const uint32_t *acc, int nq, int cps_log2,
                                            int64_t doc0, int grp, uint32_t *s_thr, uint32_t *s_off,
                                            uint32_t *s_ccnt, uint32_t *s_base, uint32_t *s_emit, uint32_t *s_maxb) {
    constexpr int NW = kUnionThreads / 64;
    const int tid = threadIdx.x, lane = gs_lane();
    const int wave = gs_uniform(tid >> 6);
    const int cps = 1 << cps_log2;
    const int nce = nq << cps_log2;  // <= kEmitChunks
    (void)tid;
    auto scan4 = [&](int ch, uint32_t vv[4], bool keep[4], uint64_t mk[4]) {
        const int g = ch >> cps_log2;
        const int thr = (int)s_thr[g];
        const uint4 v4 = *reinterpret_cast<const uint4 *>(acc + ((size_t)ch << 8) + 4 * lane);
        vv[0] = v4.x;
        vv[1] = v4.y;
        vv[2] = v4.z;
        vv[3] = v4.w;
        uint32_t tot = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            keep[u] = (int32_t)vv[u] >= thr;
            mk[u] = __ballot(keep[u]);
            tot += (uint32_t)__popcll(mk[u]);
        }
        return tot;
    };
    // Pass 1 reads a wave's chunks kEmitReads at a time, so that many LDS reads
    // are in flight instead of one read-wait-count round trip per chunk; lane g
    // holds slot g's threshold (a group holds at most 32 queries).
    {
        const int thr_l = lane < nq ? (int)s_thr[lane] : 0;
        for (int c0 = wave; c0 < nce; c0 += NW * kEmitReads) {
            uint4 v4[kEmitReads];
#pragma unroll
            for (int u = 0; u < kEmitReads; ++u) {  // past the end: the last chunk again, not counted
                const int ch = min(c0 + u * NW, nce - 1);
                v4[u] = *reinterpret_cast<const uint4 *>(acc + ((size_t)ch << 8) + 4 * lane);
            }
#pragma unroll
            for (int u = 0; u < kEmitReads; ++u) {
                const int ch = c0 + u * NW;
                if (ch >= nce) break;
                const int thr = __builtin_amdgcn_readlane(thr_l, ch >> cps_log2);
                const uint32_t cnt = (uint32_t)__popcll(__ballot((int32_t)v4[u].x >= thr)) +
                                     (uint32_t)__popcll(__ballot((int32_t)v4[u].y >= thr)) +
                                     (uint32_t)__popcll(__ballot((int32_t)v4[u].z >= thr)) +
                                     (uint32_t)__popcll(__ballot((int32_t)v4[u].w >= thr));
                if (lane == 0) {
                    s_off[ch] = cnt;
                    s_ccnt[ch] = cnt;
                }
            }
        }
    }
    __syncthreads();
    for (int g = wave; g < nq; g += NW) {
        const uint32_t c = lane < cps ? s_off[(g << cps_log2) + lane] : 0u;
        const uint32_t inc = gs_wave_incl_scan(c);
        const uint32_t run = (uint32_t)__shfl((int)inc, 63, 64);
        if (lane < cps) s_off[(g << cps_log2) + lane] = inc - c;
        if (lane == 0) {
            s_base[g] = run ? atomicAdd(a.cnt + grp * a.G + g, run) : 0u;
            s_emit[g] = run;
            s_maxb[g] = 0;
        }
    }
    __syncthreads();
    const int my_ch = wave + lane * NW;
    uint64_t live = __ballot(my_ch < nce && s_ccnt[min(my_ch, kEmitChunks - 1)] != 0);
    while (live) {
        const int ch = wave + (__ffsll((unsigned long long)live) - 1) * NW;
        live &= live - 1;
        uint32_t vv[4];
        bool keep[4];
        uint64_t mk[4];
        scan4(ch, vv, keep, mk);
        const int g = ch >> cps_log2;
        const int d = ((ch & (cps - 1)) << 8) + 4 * lane;
        const int q = grp * a.G + g;
        uint32_t base = s_base[g] + s_off[ch];
        uint32_t mb = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (keep[u]) {
                const uint32_t slot = base + (uint32_t)__popcll(mk[u] & gs_lanemask_lt());
                if (slot < (uint32_t)a.cap) {
                    a.cand_doc[(int64_t)q * a.cap + slot] = (uint32_t)(doc0 + d + u);
                    a.cand_key[(int64_t)q * a.cap + slot] = vv[u];
                }
                const uint32_t b = gs_bin_of((float)vv[u]);
                atomicAdd(a.hist + (int64_t)q * GS_HIST_BINS + b, 1u);
                mb = b > mb ? b : mb;
            }
            base += (uint32_t)__popcll(mk[u]);
        }
        if (mb) atomicMax(&s_maxb[g], mb);  // lanes holding candidates
    }
    __syncthreads();
    // tau is recomputed from the histogram when a slot's candidate count crosses
    // a multiple of max(k / 8, 64) at or above k; otherwise only the max bin is
    // published
    const uint32_t step = (uint32_t)max(a.k >> 3, 64);
    for (int g = wave; g < nq; g += NW) {
        const uint32_t e = s_emit[g];
        if (!e) continue;
        const int q = grp * a.G + g;
        const uint32_t c0 = s_base[g], c1 = c0 + e;
        const bool raise = c1 >= (uint32_t)a.k && (c0 < (uint32_t)a.k || c0 / step != c1 / step);
        if (!raise) {
            if (lane == 0) atomicMax(a.maxbin + q, s_maxb[g]);
            continue;
        }
        uint32_t top = 0;
        if (lane == 0) top = atomicMax(a.maxbin + q, s_maxb[g]);
        top = __shfl(top, 0, 64);
        top = top > s_maxb[g] ? top : s_maxb[g];
        raise_tau(a.tau + q, a.hist + (int64_t)q * GS_HIST_BINS, top, a.k);
    }
}

// One workgroup = one doc tile x one query group; the G query slices of the
// tile live in LDS as int32.  Per batch of union terms, every thread fetches one
// term's posting sub-range for the tile and its chunk count (64 * UNROLL
// postings per chunk), and the batch's (slot, weight) entries are copied to LDS.
// Waves then take chunks round-robin, load each posting once and add its
// fixed-point contribution to every query slot of the term with ds_add_u32.
// Afterwards the slices are scanned for candidates.
// PK: postings come from the packed scoring copy (gs_pack_postings): one word
// per posting with the doc's byte offset in a slice and the integer weight,
// instead of the doc id and weight arrays.
// HD: the slices start from the coarse heavy-term sums (k_head_scores) instead
// of zero, and the group's union holds the other terms only.
template <int WT, int UNROLL, bool PK, bool SE, bool HD>
__global__ void __launch_bounds__(kUnionThreads, HD ? 4 : 2) k_score_union(const UnionArgs a) {
    using W = gs_weight<WT>;
    using store_t = typename W::store_t;
    using pk_t = uint32_t;
    constexpr int CH = 64 * UNROLL;
    constexpr int NW = kUnionThreads / 64;

    extern __shared__ __align__(16) unsigned char lds_raw[];
    __shared__ int32_t s_scan[kUnionThreads / 64 + 1];
    __shared__ uint32_t s_thr[32], s_emit[32], s_maxb[32], s_base[32], s_mfix[32];
    __shared__ uint32_t s_lhist[kLocalSlots][kLocalBins];
    __shared__ uint32_t s_off[kEmitChunks], s_ccnt[kEmitChunks];

    const int tid = threadIdx.x, lane = gs_lane();
    const int wave = gs_uniform(tid >> 6);
    const int64_t lin = (int64_t)(blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
    const int n_blk = (a.tiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
    if (lin >= (int64_t)n_blk * a.n_groups) return;
    const int blk = (int)(lin / a.n_groups);
    const int grp = (int)(lin % a.n_groups);
    const int tile_lo = a.tile_begin + blk * a.tiles_per_wg;
    const int tile_hi = min(tile_lo + a.tiles_per_wg, a.tile_begin + a.tiles);
    const int nq = min(a.G, a.B - grp * a.G);
    const int slice_shift = a.tile_log2 + 2;  // bytes per query slice = 1 << slice_shift

    uint32_t *acc = reinterpret_cast<uint32_t *>(lds_raw);
    int64_t *s_start = reinterpret_cast<int64_t *>(lds_raw + ((size_t)a.G << slice_shift));
    int32_t *s_len = reinterpret_cast<int32_t *>(s_start + kUnionBatch);
    int32_t *s_cst = s_len + kUnionBatch;    // [kUnionBatch + 1], s_cst[nb] = total chunks
    int32_t *s_e = s_cst + kUnionBatch + 1;  // [kUnionBatch], (entry count << 16 | first entry) per term
    int64_t *s_toff = reinterpret_cast<int64_t *>(s_e + kUnionBatch + 3);  // [kUnionBatch] list offsets (8-aligned)
    int32_t *s_tid = reinterpret_cast<int32_t *>(s_toff + kUnionBatch);    // [kUnionBatch] term ids

    const int64_t row = (int64_t)a.n_tiles + 1;
    const int32_t *uterm = a.u_term + (int64_t)grp * a.ecap;
    const int32_t *uebeg = a.u_ebeg + (int64_t)grp * (a.ecap + 1);
    // The group's first union terms are loaded together with their count (the
    // loads stay inside the group's rows; entries past the count are not used),
    // so the bounds below wait for one load instead of two in a row.
    int32_t t_first = 0, e_first = 0;
    if (tid < min(kUnionBatch, a.ecap)) {
        t_first = uterm[tid];
        e_first = uebeg[tid];
    }
    const int U = a.u_count[grp];
    const uint2 *esw = a.e_sw + (int64_t)grp * a.ecap;
    const store_t *wall = reinterpret_cast<const store_t *>(a.w);
    const pk_t *pkd = reinterpret_cast<const pk_t *>(a.pk);

    // The first tile's slices are set while the term loads are in flight: zero,
    // or the 12-bit coarse heavy-term sums c as c * 2^kHeadShift.  Those come as
    // 8-doc pieces of the block-major k_head_scores rows (8 high bytes and 4
    // bytes of low nibbles), at most kHeadPieces per thread (G * tile = 16 Ki
    // docs), loaded for the next tile before the current tile's emission.  (A
    // thread's 8 docs are 32 bytes of its slice, as with 16-bit sums: 16-doc
    // pieces, 64 bytes per thread, doubled the bank conflicts of the slices'
    // set-up.)
    constexpr int kHeadPieces = (int)(kUnionTileLds / 4 / 8 / kUnionThreads);
    uint2 hp[HD ? kHeadPieces : 1];
    uint32_t hn[HD ? kHeadPieces : 1];
    auto load_head = [&](int tile) {
        if constexpr (HD) {
            const int per_log2 = a.tile_log2 - 3;  // 8-doc pieces per slot of a tile
            const int64_t doc0 = (int64_t)tile << a.tile_log2;
#pragma unroll
            for (int u = 0; u < kHeadPieces; ++u) {
                const int i = tid + u * kUnionThreads;
                if (i < (nq << per_log2)) {
                    const int g = i >> per_log2;
                    const int64_t d = doc0 + ((int64_t)(i & ((1 << per_log2) - 1)) << 3);
                    const uint8_t *rp = a.hsc + ((d / kHeadBlock) * a.hsc_ld + grp * a.G + g) * kHscRow;
                    const int o = (int)(d % kHeadBlock);
                    // read once: non-temporal loads keep the L2 for the posting words
                    // (scoring 5.57 vs 5.65 ms at C3)
                    const gs_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const gs_u32x2 *>(rp + o));
                    hp[u] = make_uint2(v.x, v.y);
                    hn[u] = __builtin_nontemporal_load(
                        reinterpret_cast<const uint32_t *>(rp + kHeadBlock + (o >> 1)));
                }
            }
        } else {
            (void)tile;
        }
    };
    auto zero_slices = [&]() {
        uint4 *z = reinterpret_cast<uint4 *>(acc);
        if constexpr (HD) {
            // c * 2^20 = (high byte << 24) | (low nibble << 20): per doc one
            // v_perm_b32 placing the high byte at byte 3 and the nibble's byte at
            // byte 2 (shifted up by 4 for the even doc's low nibble), and one and
            // clearing the other nibble (bits 16..19)
            static_assert(kHeadShift == 20, "slices take the coarse sums' bits in place");
#pragma unroll
            for (int u = 0; u < kHeadPieces; ++u) {
                const int i = tid + u * kUnionThreads;
                if (i < (nq << (a.tile_log2 - 3))) {
                    const uint32_t hw[2] = {hp[u].x, hp[u].y};
                    const uint32_t nw = hn[u], nl = nw << 4;
#pragma unroll
                    for (int q4 = 0; q4 < 2; ++q4) {  // docs 4 q4 .. 4 q4 + 3 of the piece
                        const uint32_t j0 = 2u * (uint32_t)q4;  // their nibbles' bytes j0, j0 + 1
                        z[2 * i + q4] = make_uint4(
                            __builtin_amdgcn_perm(hw[q4], nl, 0x04000C0Cu | (j0 << 16)) & 0xFFF00000u,
                            __builtin_amdgcn_perm(hw[q4], nw, 0x05000C0Cu | (j0 << 16)) & 0xFFF00000u,
                            __builtin_amdgcn_perm(hw[q4], nl, 0x06000C0Cu | ((j0 + 1) << 16)) & 0xFFF00000u,
                            __builtin_amdgcn_perm(hw[q4], nw, 0x07000C0Cu | ((j0 + 1) << 16)) & 0xFFF00000u);
                    }
                }
            }
        } else {
            const int n16 = (nq << slice_shift) >> 4;
            for (int i = tid; i < n16; i += kUnionThreads) z[i] = make_uint4(0, 0, 0, 0);
        }
    };
    load_head(tile_lo);
    zero_slices();

    // A group whose union fits one batch describes its terms in LDS once (term
    // id, list offset, entry range); thread `term` holds the term's bounds in the
    // current tile and loads the next tile's while the current one is scored.
    const bool single = U <= kUnionBatch;
    int my_lo = 0, my_hi = 0;
    if (single && tid < U) {
        const int32_t t = t_first;
        s_tid[tid] = t;
        s_toff[tid] = a.offsets[t];
        s_e[tid] = e_first;
        my_lo = a.tb[(int64_t)t * row + tile_lo];
        my_hi = a.tb[(int64_t)t * row + tile_lo + 1];
    }
    if (tid < nq) s_mfix[tid] = a.mfix[grp * a.G + tid];

    for (int tile = tile_lo; tile < tile_hi; ++tile) {
    const int64_t doc0 = (int64_t)tile << a.tile_log2;
    // tau of the group's queries, read now so that its latency hides behind the
    // scoring (tau only rises: an older value admits more candidates, never fewer)
    uint32_t r_tau = 0;
    if (tid < nq) r_tau = gs_load_relaxed(a.tau + grp * a.G + tid);
    if (tile > tile_lo) {
        __syncthreads();  // the previous tile's emission is done with the slices
        zero_slices();
    }

    for (int b0 = 0; b0 < U; b0 += kUnionBatch) {
        const int nb = min(kUnionBatch, U - b0);
        __syncthreads();  // LDS zeroed / previous batch consumed
        int nch = 0;
        if (tid < nb) {
            int lo, hi;
            if (single) {
                lo = my_lo;
                hi = my_hi;
                s_start[tid] = s_toff[tid] + lo;
                if (tile + 1 < tile_hi) {  // prefetch the next tile's bounds
                    const int32_t *bt = a.tb + (int64_t)s_tid[tid] * row + tile + 1;
                    my_lo = bt[0];
                    my_hi = bt[1];
                }
            } else {
                const int32_t t = uterm[b0 + tid];
                const int32_t *bt = a.tb + (int64_t)t * row + tile;
                lo = bt[0];
                hi = bt[1];
                s_start[tid] = a.offsets[t] + lo;
                s_e[tid] = uebeg[b0 + tid];
            }
            s_len[tid] = hi - lo;
            nch = (hi - lo + CH - 1) / CH;
        }
        // exclusive scan of chunk counts
        int x = nch;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(x, d, 64);
            if (lane >= d) x += o;
        }
        if (lane == 63) s_scan[wave] = x;
        __syncthreads();
        if (tid == 0) {
            int accs = 0;
            for (int w = 0; w < NW; ++w) {
                const int s = s_scan[w];
                s_scan[w] = accs;
                accs += s;
            }
            s_scan[NW] = accs;
        }
        __syncthreads();
        if (tid < nb) s_cst[tid] = s_scan[wave] + x - nch;
        const int total = s_scan[NW];
        if (tid == 0) s_cst[nb] = total;
        __syncthreads();

        // Chunk loop.  A chunk is 64 * UNROLL consecutive postings of one union
        // term inside the tile; wave w takes chunks w, w + NW, ...  Each wave first
        // describes its next 64 chunks, one per lane (term found by binary search
        // over the chunk scan), so the loop itself reads no LDS: chunk fields come
        // from v_readlane, and the postings come from buffer loads issued one chunk
        // ahead (the term's (slot, weight) entries from scalar loads, or for groups
        // of more than 4 queries a buffer load, issued with them).  The loads go
        // through per-chunk buffer resources sized to the chunk, so every lane uses
        // the same byte offset register (lane * size, plus an immediate per posting
        // group) and lanes past the chunk's end read 0.
        struct Chunk {
            int n, m, e0;
            uint32_t b0, w0, b1, w1;  // SE: the term's first two entries: slice byte offset - doc0 * 4, weight
            uint32_t badj, my_w;      // !SE: lane j: the j-th entry's slice byte offset - doc0 * 4, weight
            int32_t doc[UNROLL];
            store_t wv[UNROLL];
        };
        // A wave raises its issue priority as its share of the chunks completes
        // (0 for the first quarter, then 1, 2, 3).  The two workgroups of a CU
        // share its SIMDs: serving the waves that are further along first keeps
        // the workgroups apart, so that one's emission and set-up overlap the
        // other's adds.  (Lowering it instead, 3, 2, 1, 0, evened out the waves
        // of a workgroup but drew the two workgroups into step.)  The hybrid
        // search's adds, a smaller part of its work in many short chunks, stay
        // at priority 0 with no per-chunk bookkeeping: C3 scoring 5.30-5.35 vs
        // 5.52-5.58 ms with the raising (5.48 with the levels counted but not set).
        const int my_total = (total - wave + NW - 1) / NW;  // chunks of this wave in the batch
        // level = floor(4 done / my_total), i.e. level >= L once done >= ceil(L
        // my_total / 4); only the next boundary is compared per chunk
        auto quarter = [&](int L) { return (L * my_total + 3) >> 2; };
        int level = 0, next_at = quarter(1);
        __builtin_amdgcn_s_setprio(0);
        auto progress = [&](int done) {
            if constexpr (HD) return;
            if (done < next_at) return;
            while (level < 3 && done >= quarter(level + 1)) ++level;
            next_at = level < 3 ? quarter(level + 1) : 0x7FFFFFFF;
            if (level == 1) __builtin_amdgcn_s_setprio(1);
            else if (level == 2) __builtin_amdgcn_s_setprio(2);
            else __builtin_amdgcn_s_setprio(3);
        };
        for (int cb = wave; cb < total; cb += 64 * NW) {
            const int nmine = min(64, (total - cb + NW - 1) / NW);  // chunks of this wave in the block
            int64_t md_p0 = 0;
            int md_n = 0, md_e0 = 0, md_m = 0;
            // packed copy: lane c also holds its chunk's load window as the
            // fetch needs it (base address of the 64-posting-aligned window, the
            // chunk's offset in it, its posting and entry counts), so the fetch
            // does no 64-bit address arithmetic
            uint32_t md_blo = 0, md_bx = 0, md_nm = 0;
            {
                const int c = cb + lane * NW;
                if (c < total) {
                    int lo = 0, hi = nb;  // s_cst[lo] <= c < s_cst[hi]
                    while (hi - lo > 1) {
                        const int mid = (lo + hi) >> 1;
                        if (s_cst[mid] <= c) lo = mid;
                        else hi = mid;
                    }
                    const int ci = c - s_cst[lo];
                    md_p0 = s_start[lo] + (int64_t)ci * CH;
                    md_n = min(CH, s_len[lo] - ci * CH);
                    md_e0 = s_e[lo] & 0xFFFF;
                    md_m = s_e[lo] >> 16;
                    if constexpr (PK) {
                        const int64_t pb = md_p0 & ~int64_t(63);
                        const uint64_t addr = (uint64_t)(uintptr_t)(pkd + pb);  // < 2^48 (packed_usable)
                        md_blo = (uint32_t)addr;
                        md_bx = (uint32_t)(addr >> 32) | ((uint32_t)(md_p0 - pb) << 16);
                        md_nm = (uint32_t)md_n | ((uint32_t)md_m << 16);
                    }
                }
            }
            // byte address of doc d in the slice at LDS offset `base`: (d << 2) +
            // base - (doc0 << 2), in wrapping 32-bit arithmetic (one v_add per add);
            // packed postings carry (d - doc0) << 2 already
            const uint32_t doc0_4 = PK ? 0u : (uint32_t)doc0 << 2;
            auto fetch = [&](int j, Chunk &k) {
                if constexpr (PK) {
                    const uint32_t blo = (uint32_t)__builtin_amdgcn_readlane((int)md_blo, j);
                    const uint32_t bx = (uint32_t)__builtin_amdgcn_readlane((int)md_bx, j);
                    const uint32_t nm = (uint32_t)__builtin_amdgcn_readlane((int)md_nm, j);
                    k.n = (int)(nm & 0xFFFFu);
                    k.m = (int)(nm >> 16);
                    k.e0 = __builtin_amdgcn_readlane(md_e0, j);
                    if constexpr (SE) {  // entries as in the general path below (packed: doc0_4 = 0)
                        typedef const __attribute__((address_space(4))) uint32_t *const_u32_p;
                        const const_u32_p ep = (const_u32_p)(uintptr_t)(esw + k.e0);
                        k.b0 = ep[0] << slice_shift;
                        k.w0 = ep[1];
                        k.b1 = ep[2] << slice_shift;
                        k.w1 = ep[3];
                    } else {
                        const uint2 sw = gs_bload64(gs_rsrc(esw + k.e0, (uint32_t)k.m * 8u), lane * 8);
                        k.badj = sw.x << slice_shift;
                        k.my_w = sw.y;
                    }
                    const int sh = (int)(bx >> 16);
                    const pk_t *base = reinterpret_cast<const pk_t *>((uintptr_t)(((uint64_t)(bx & 0xFFFFu) << 32) | blo));
                    const auto rp = gs_rsrc(base, (uint32_t)(sh + k.n) * (uint32_t)sizeof(pk_t));
                    const int o_p = (lane + sh) * (int)sizeof(pk_t);
#pragma unroll
                    for (int u = 0; u < UNROLL; ++u) k.doc[u] = (int32_t)gs_bload32(rp, o_p + u * 256);
                    return;
                }
                const int64_t p0 = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(md_p0 >> 32), j) << 32) |
                                             (uint32_t)__builtin_amdgcn_readlane((int)md_p0, j));
                k.n = __builtin_amdgcn_readlane(md_n, j);
                k.m = __builtin_amdgcn_readlane(md_m, j);
                k.e0 = __builtin_amdgcn_readlane(md_e0, j);
                if constexpr (SE) {
                    // Groups of at most 4 slots: the term's first two (slot, weight)
                    // entries arrive in SGPRs by one scalar load (read-only here; the
                    // entry array has one entry of padding, so the pair never leaves
                    // it); further ones are read one by one in add_entries.
                    typedef const __attribute__((address_space(4))) uint32_t *const_u32_p;
                    const const_u32_p ep = (const_u32_p)(uintptr_t)(esw + k.e0);
                    k.b0 = (ep[0] << slice_shift) - doc0_4;
                    k.w0 = ep[1];
                    k.b1 = (ep[2] << slice_shift) - doc0_4;
                    k.w1 = ep[3];
                } else {
                    // larger groups: lane j loads entry j (a scalar load per entry
                    // would wait on the LDS adds issued before it)
                    const uint2 sw = gs_bload64(gs_rsrc(esw + k.e0, (uint32_t)k.m * 8u), lane * 8);
                    k.badj = (sw.x << slice_shift) - doc0_4;
                    k.my_w = sw.y;
                }
                // The resources start at p0 rounded down to 64 postings; the lane
                // offset carries the remainder.  It changes per chunk, so it is
                // computed here and the per-group constants fold into the loads'
                // immediate offsets.
                const int64_t pb = p0 & ~int64_t(63);
                const int sh = (int)(p0 - pb);
                if constexpr (PK) {
                    const auto rp = gs_rsrc(pkd + pb, (uint32_t)(sh + k.n) * (uint32_t)sizeof(pk_t));
                    const int o_p = (lane + sh) * (int)sizeof(pk_t);
#pragma unroll
                    for (int u = 0; u < UNROLL; ++u) k.doc[u] = (int32_t)gs_bload32(rp, o_p + u * 256);
                } else {
                    const auto rd = gs_rsrc(a.doc + pb, (uint32_t)(sh + k.n) * 4u);
                    const auto rw = gs_rsrc(wall + pb, (uint32_t)(sh + k.n) * (uint32_t)sizeof(store_t));
                    const int o_doc = (lane + sh) * 4, o_w = (lane + sh) * (int)sizeof(store_t);
#pragma unroll
                    for (int u = 0; u < UNROLL; ++u) {
                        k.doc[u] = (int32_t)gs_bload32(rd, o_doc + u * 256);
                        k.wv[u] = W::bload(rw, o_w + u * 64 * (int)sizeof(store_t));
                    }
                }
            };
            // the first NG 64-posting groups of a chunk, added to one query slot
            auto add_groups = [&](const Chunk &k, auto ngc, uint32_t badj, uint32_t wb) {
                constexpr int NG = decltype(ngc)::value;
#pragma unroll
                for (int u = 0; u < NG; ++u) {
                    const uint32_t d = (uint32_t)k.doc[u];
                    if constexpr (!PK)
                        lds_add<uint32_t>(reinterpret_cast<uint32_t *>(lds_raw + ((d << 2) + badj)),
                                          fixed_contrib<WT>(wb, k.wv[u]));
                    else
                        lds_add<uint32_t>(reinterpret_cast<uint32_t *>(lds_raw + ((d & 0xFFFFu) + badj)),
                                          packed_contrib<WT>(wb, d));
                }
            };
            // every entry (query slot) of the chunk's term; the group count is
            // resolved once per chunk, so the entry loop is straight-line adds
            auto add_entries = [&](const Chunk &k, auto ngc) {
                if constexpr (SE) {
                    add_groups(k, ngc, k.b0, k.w0);
                    if (k.m > 1) add_groups(k, ngc, k.b1, k.w1);
                    for (int e = 2; e < k.m; ++e) {
                        const uint2 sw = esw[k.e0 + e];
                        add_groups(k, ngc, (sw.x << slice_shift) - doc0_4, sw.y);
                    }
                } else {
                    for (int e = 0; e < k.m; ++e)
                        add_groups(k, ngc, (uint32_t)__builtin_amdgcn_readlane((int)k.badj, e),
                                   (uint32_t)__builtin_amdgcn_readlane((int)k.my_w, e));
                }
            };
            auto apply = [&](Chunk &k, int j) {
                // One wait for the whole chunk: its loads are all but the newest
                // vm ones (the next chunk's, issued by the fetch before this call),
                // so the adds below need no per-group waits.
                {
                    constexpr int vm = (PK ? UNROLL : 2 * UNROLL) + (SE ? 0 : 1);
                    static_assert(vm < 64, "vmcnt is 6 bits");
                    __builtin_amdgcn_s_waitcnt((vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | (0xF << 8));
                }
                if (k.m > 64) {  // a term held by more than 64 query slots (queries repeating terms)
                    if (k.n < CH)
#pragma unroll
                        for (int u = 0; u < UNROLL; ++u)
                            k.doc[u] = u * 64 + lane < k.n ? k.doc[u] : (PK ? lane << 2 : (int32_t)doc0 + lane);
                    const int e0 = __builtin_amdgcn_readlane(md_e0, j);
                    for (int e = e0; e < e0 + k.m; ++e)
                        add_groups(k, std::integral_constant<int, UNROLL>{}, (esw[e].x << slice_shift) - doc0_4,
                                   esw[e].y);
                    return;
                }
                if (k.n == CH) {
                    add_entries(k, std::integral_constant<int, UNROLL>{});
                    return;
                }
                // last chunk of a term: only the 64-posting groups holding postings
                // run, and in the last of them lanes past the end read weight 0 and
                // are sent to doc doc0 + lane, a word of their own (one shared word
                // would serialise their atomics; a packed lane gets offset lane * 4
                // and weight 0)
                gs_dispatch_upto<UNROLL>((k.n + 63) >> 6, [&](auto ngc) {
                    constexpr int L = decltype(ngc)::value - 1;
                    k.doc[L] = L * 64 + lane < k.n ? k.doc[L] : (PK ? lane << 2 : (int32_t)doc0 + lane);
                    add_entries(k, ngc);
                });
            };
            // two chunk buffers in rotation: the loads of the wave's next chunk are
            // in flight while the current one is applied.  Fetches past the end
            // re-read the last chunk (unconditional fetches keep the wait counts
            // static).
            Chunk ka, kb;
            const int last = nmine - 1;
            const int done0 = (cb - wave) / NW;  // chunks this wave applied in earlier blocks
            int j = 0;
            fetch(0, ka);
            while (true) {
                fetch(min(j + 1, last), kb);
                progress(done0 + j);
                apply(ka, j);
                if (++j > last) break;
                fetch(min(j + 1, last), ka);
                progress(done0 + j);
                apply(kb, j);
                if (++j > last) break;
            }
        }
    }
    // Emission and the next tile's set-up are latency-bound: they issue at the
    // highest priority, ahead of the other workgroup's adds.
    __builtin_amdgcn_s_setprio(3);
    if (tile + 1 < tile_hi) load_head(tile + 1);
    __syncthreads();

    // ---- emission of candidates >= tau - margin (emit_slices), the seed
    // launch's thresholds first raised to the slots' local k-th scores
    const int cps_log2 = a.tile_log2 - 8;  // 256-doc chunks per slice = 1 << cps_log2
    const int nce = nq << cps_log2;        // <= kEmitChunks (G * TILE <= kUnionTileLds / 4)
    if (tid < nq) s_thr[tid] = emit_threshold(r_tau, s_mfix[tid]);
    if (a.local_k > 0 && nq <= kLocalSlots) {
        // Seed launch (tau = 0): every positive doc would be a candidate.  Any k
        // docs of this tile scoring >= X bound the query's k-th score from below
        // by X, so the slot's local k-th score L gives the threshold L - margin.
        // L is bounded from below by the lower edge of the histogram bin (linear
        // over (0, slot max]) where the count from the top reaches k.
        if (tid < nq) s_maxb[tid] = 0;
        for (int i = tid; i < kLocalSlots * kLocalBins; i += kUnionThreads) (&s_lhist[0][0])[i] = 0;
        __syncthreads();
        for (int ch = wave; ch < nce; ch += NW) {
            const uint4 v4 = *reinterpret_cast<const uint4 *>(acc + ((size_t)ch << 8) + 4 * lane);
            const int mx = max(max((int32_t)v4.x, (int32_t)v4.y), max((int32_t)v4.z, (int32_t)v4.w));
            const uint32_t wm = gs_wave_max_u32((uint32_t)max(mx, 0));
            if (lane == 0 && wm) atomicMax(&s_maxb[ch >> cps_log2], wm);
        }
        __syncthreads();
        for (int ch = wave; ch < nce; ch += NW) {
            const int g = ch >> cps_log2;
            const uint64_t span = (uint64_t)s_maxb[g] + 1;
            const uint4 v4 = *reinterpret_cast<const uint4 *>(acc + ((size_t)ch << 8) + 4 * lane);
            const uint32_t vs[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if ((int32_t)vs[u] > 0) atomicAdd(&s_lhist[g][(uint64_t)vs[u] * kLocalBins / span], 1u);
        }
        __syncthreads();
        for (int g = wave; g < nq; g += NW) {  // lane l: bins 255 - 4l .. 252 - 4l
            uint32_t c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) sum += (c[j] = s_lhist[g][kLocalBins - 1 - 4 * lane - j]);
            const uint32_t inc = gs_wave_incl_scan(sum);
            const uint64_t hit = __ballot(inc >= (uint32_t)a.local_k);
            if (hit) {
                const int l = __ffsll((unsigned long long)hit) - 1;
                if (lane == l) {
                    uint32_t cum = inc - sum;
                    int j = 0;
                    while (cum + c[j] < (uint32_t)a.local_k) cum += c[j++];
                    const uint64_t b = (uint64_t)(kLocalBins - 1 - 4 * lane - j);
                    const uint64_t span = (uint64_t)s_maxb[g] + 1;
                    const uint32_t edge = (uint32_t)((b * span + kLocalBins - 1) / kLocalBins);  // least v of bin b
                    const uint32_t t = emit_threshold(edge, s_mfix[g]);
                    if (t > s_thr[g]) s_thr[g] = t;
                }
            }
        }
        __syncthreads();
        if (tid < nq) s_maxb[tid] = 0;
    }
    __syncthreads();
    const EmitArgs ea{a.tau, a.cnt, a.maxbin, a.hist, a.cand_doc, a.cand_key, a.G, a.cap, a.k};
    emit_slices(ea, acc, nq, cps_log2, doc0, grp, s_thr, s_off, s_ccnt, s_base, s_emit, s_maxb);
    }  // tile
}

// ---------------------------------------------------------------------- heavy terms on the MFMA units

// The heavy terms (the index's GS_HEAVY_TERMS longest lists) hold most of the
// postings a batch scores: at C3 the 64 longest lists carry 91% of the scored
// postings, the 128 longest 96%.  The hybrid search computes their part of every
// (query, doc) sum with int8 matrix products (k_head_scores) and starts each
// LDS slice of k_score_union from it; the slices then take the other ("tail")
// terms' postings as LDS adds.
//
// Exactness.  A tail occurrence j adds qi_j * wq (qi_j = rint(q_j 2^f), wq the
// packed copy's integer weight), as in the LDS-add search; a heavy term h
// contributes 2^r a_h wq with a_h = sum over the query's occurrences of h of
// rint(q_j 2^(f - r)), |a_h| <= 16383 (k_query_prep_hybrid picks f and the
// query's shift r and bounds the error).  With a_h = 128 ah + al and wq = 128 wh
// + wl (al, wl in [0, 127], ah, wh signed bytes):
//   sum_h a_h wq_h = sum al wl + 2^7 (sum al wh + sum ah wl) + 2^14 sum ah wh,
// four chains of v_mfma_i32_16x16x64_i8 per 16 docs x 16 queries, one product
// per 64 heavy terms in each, every one an exact int32 sum (|.| <= 2 * 256 * 128
// * 128 = 2^23 for the middle one over 256 terms); the combination H is exact in
// wrapping 32-bit arithmetic because it fits int32.  The slices start from
// floor(H / 2^20) * 2^20, which is below H by less than 2^20: the margin grows
// by 2^20 (k_query_prep_hybrid), so every doc that can reach the top k is still
// rescored in fp64, and the answers stay exact.  (|H| < 2^31, so floor(H / 2^20)
// takes 12 bits: bits 20..31 of H, the slice's start being H & 0xFFF00000.)


typedef int32_t gs_v4i __attribute__((ext_vector_type(4)));

// Coarse heavy-term sums of every (slot, doc): c = floor(H(s, d) / 2^20), 12
// bits (|H| < 2^31), in rows of kHscRow bytes per (512-doc block b, slot s),
// block-major -- row b * Bpad + s at byte (b * Bpad + s) * kHscRow -- so that
// each workgroup writes one contiguous run, slots 0..Bpad-1 (slots past B hold
// zero limbs).  A row holds its 512 docs' high bytes (bits 4..11 of c; doc d mod
// 512 at byte d mod 512), then their low nibbles (bits 0..3 of c), two per
// byte: doc d mod 512 at byte 512 + (d mod 512) / 2, in the low nibble for even
// d.  Blocks past the head rows (docs past the collection) hold zeros.
//
// Eight waves, each holding its 4 blocks of 16 docs as the A operands (per 64
// heavy terms: lane = doc lane % 16, terms 16 (lane / 16) .. + 15, two limbs)
// for every block of 16 slots (B operands: the query limbs, same lane layout,
// loaded one block ahead).  A lane's 4 outputs are 4 consecutive docs of one
// slot (rows 4 (lane / 16) + i, column lane % 16 of the 16x16 product); their
// high half-words (bits 16..31 of H) go to an LDS stage of the 16 slots' rows
// (double-buffered, rows padded so that the 16 rows of a store fall in
// different banks).  The workgroup then writes the rows out, 8 docs per thread
// and step as 8 high bytes and 4 bytes of nibbles: one contiguous 12 KiB run
// per block of slots.  (Packing the 12 bits before the stage held the kernel at
// 84 VGPRs, two workgroups per CU instead of three.  Each wave writing its own
// 64 docs of the rows, with no workgroup barrier, measured slower; so did int8
// coarse sums with a per-query shift: fewer bytes, but their wider margin costs
// the scorer and the rescoring more than the writes save.)
constexpr int kHeadStageRow = kHeadBlock + 16;  // int16 per staged row (bank padding)

__global__ void __launch_bounds__(512) k_head_scores(const int8_t *__restrict__ head, int64_t head_rows,
                                                     const int8_t *__restrict__ alimb,
                                                     const int32_t *__restrict__ hshift, int32_t B, int32_t Bpad,
                                                     uint8_t *__restrict__ out) {
    constexpr int HT = kHeavyTerms;
    constexpr int KB = HT / 64;               // 64-term blocks of the products
    constexpr int CPW = kHeadBlock / 16 / 8;  // blocks of 16 docs per wave
    __shared__ __align__(16) int16_t stage[2][16 * kHeadStageRow];
    const int lane = gs_lane(), tid = threadIdx.x;
    const int wave = gs_uniform(tid >> 6);
    const int64_t doc0 = (int64_t)blockIdx.x * kHeadBlock;
    uint8_t *ob = out + (int64_t)blockIdx.x * Bpad * kHscRow;
    if (doc0 >= head_rows) {  // docs past the collection
        for (int64_t i = tid; i < (int64_t)Bpad * kHscRow / 16; i += blockDim.x)
            reinterpret_cast<uint4 *>(ob)[i] = make_uint4(0, 0, 0, 0);
        return;
    }
    gs_v4i dl[CPW][KB], dh[CPW][KB];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int8_t *hp = head + (doc0 + (wave * CPW + c) * 16 + (lane & 15)) * (2 * HT) + (lane >> 4) * 16;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            dl[c][kb] = *reinterpret_cast<const gs_v4i *>(hp + kb * 64);
            dh[c][kb] = *reinterpret_cast<const gs_v4i *>(hp + HT + kb * 64);
        }
    }
    auto load_q = [&](int rb, gs_v4i (&ql)[KB], gs_v4i (&qh)[KB], int &r) {
        const int s = rb + (lane & 15);
        const int8_t *ap = alimb + (int64_t)s * (2 * HT) + (lane >> 4) * 16;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            ql[kb] = *reinterpret_cast<const gs_v4i *>(ap + kb * 64);
            qh[kb] = *reinterpret_cast<const gs_v4i *>(ap + HT + kb * 64);
        }
        r = s < B ? hshift[s] : 0;
    };
    gs_v4i ql[KB], qh[KB];
    int r;
    load_q(0, ql, qh, r);
    // 8-doc pieces of the 16 staged rows: piece i = row * (kHeadBlock / 8) + col / 8
    constexpr int kHeadPiecesPerThread = 16 * kHeadBlock / 8 / 512;
    static_assert(kHeadPiecesPerThread * 512 == 16 * kHeadBlock / 8, "whole pieces per thread");
    for (int rb = 0, buf = 0; rb < Bpad; rb += 16, buf ^= 1) {
        gs_v4i nl[KB], nh[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            nl[kb] = ql[kb];
            nh[kb] = qh[kb];
        }
        int nr = r;
        if (rb + 16 < Bpad) load_q(rb + 16, nl, nh, nr);
        int16_t *st = stage[buf];
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            gs_v4i c00 = {0, 0, 0, 0}, cm = {0, 0, 0, 0}, c11 = {0, 0, 0, 0};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                c00 = __builtin_amdgcn_mfma_i32_16x16x64_i8(dl[c][kb], ql[kb], c00, 0, 0, 0);
                cm = __builtin_amdgcn_mfma_i32_16x16x64_i8(dh[c][kb], ql[kb], cm, 0, 0, 0);
                cm = __builtin_amdgcn_mfma_i32_16x16x64_i8(dl[c][kb], qh[kb], cm, 0, 0, 0);
                c11 = __builtin_amdgcn_mfma_i32_16x16x64_i8(dh[c][kb], qh[kb], c11, 0, 0, 0);
            }
            uint32_t w[2];
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const uint32_t h0 = ((uint32_t)c00[i] + ((uint32_t)cm[i] << 7) + ((uint32_t)c11[i] << 14)) << r;
                const uint32_t h1 =
                    ((uint32_t)c00[i + 1] + ((uint32_t)cm[i + 1] << 7) + ((uint32_t)c11[i + 1] << 14)) << r;
                // the high half-words of h0 and h1 (one v_perm_b32): bits 16..31
                w[i >> 1] = __builtin_amdgcn_perm(h1, h0, 0x07060302u);
            }
            const int d = (wave * CPW + c) * 16 + 4 * (lane >> 4);
            *reinterpret_cast<uint2 *>(st + (lane & 15) * kHeadStageRow + d) = make_uint2(w[0], w[1]);
        }
        // the stage is complete; the other one's copy-out (one block back) ended
        // before any wave got here, since it precedes this barrier in every wave
        __syncthreads();
        // 8-doc pieces tid and tid + 512 of the 16 rows.  c = bits 20..31 of H =
        // bits 4..15 of the staged half-word: its high byte, and its bits 4..7
        // as the low nibble, two docs per byte (the even doc's in the low
        // nibble).  Buffer stores into this block of slots' 12 KiB run take
        // 32-bit lane offsets: with 64-bit addresses the kernel held 92 VGPRs
        // (two workgroups per CU), and spilled one of them at 80.
        static_assert(kHeadShift == 20, "the coarse sums are bits 20..31");
        const auto rs = gs_rsrc(ob + (int64_t)rb * kHscRow, 16 * kHscRow);
#pragma unroll
        for (int j = 0; j < kHeadPiecesPerThread; ++j) {
            const uint32_t i = (uint32_t)(tid + j * 512);
            const uint32_t row = i / (kHeadBlock / 8), col = (i % (kHeadBlock / 8)) * 8;
            // docs col + 2k and col + 2k + 1 in word k
            const uint4 u = *reinterpret_cast<const uint4 *>(st + row * kHeadStageRow + col);
            const gs_u32x2 hv = {__builtin_amdgcn_perm(u.y, u.x, 0x07050301u),
                                 __builtin_amdgcn_perm(u.w, u.z, 0x07050301u)};
            auto nib2 = [](uint32_t v) { return ((v >> 4) & 0x0Fu) | ((v >> 16) & 0xF0u); };
            const uint32_t nb = nib2(u.x) | (nib2(u.y) << 8) | (nib2(u.z) << 16) | (nib2(u.w) << 24);
            __builtin_amdgcn_raw_buffer_store_b64(hv, rs, (int)(row * kHscRow + col), 0, 0);  // 8 high bytes
            __builtin_amdgcn_raw_buffer_store_b32(nb, rs, (int)(row * kHscRow + kHeadBlock + col / 2), 0, 0);
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            ql[kb] = nl[kb];
            qh[kb] = nh[kb];
        }
        r = nr;
    }
}

// Query prep of the hybrid search: one wave per slot (slots past B, up to the
// multiple of 16, get zero limbs).  As k_query_prep, plus the heavy terms' limbs and shift.  Float
// weights (packed copy, pk_shift = s, W_t = rint(max|w(t)| 2^s)):
//  * tail occurrence j: qi_j = rint(q_j 2^f), |qi_j| < 2^23 (v_mul_i32_i24);
//  * heavy term h: a_h = sum over its occurrences of rint(q_j 2^(f - r)),
//    |a_h| <= 16383 (two limbs), contributing 2^r a_h wq;
//  * per product the error is <= W_t / 2 + |q| 2^f / 2 (tail) or
//    2^(r-1) W_t + |q| 2^f / 2 (heavy), so a doc's sum is within
//    E = Bw_t / 2 + 2^(r-1) Bw_h + Q 2^f / 2 of exact in fixed-point units
//    (scale 2^(f+s)), and sum |contributions| <= A 2^f + Bw_t / 2 + 2^(r-1) Bw_h,
//    A = sum_j |q_j| W_j (1 + dup), Bw_* = sum W_j (1 + dup) over tail / heavy
//    occurrences, Q = sum |q_j| (1 + dup);
//  * f is the largest exponent keeping that below 2^31 and the tail operands
//    below 2^23, with r the smallest shift keeping every a_h in range (from
//    s_h = sum of |q_j| over h's occurrences); the margin is k_query_prep's for
//    this E, plus 2^kHeadShift for the coarse heavy-term start of the slices.
// A query without feasible (f, r), or whose limbs do not fit after all, gets
// mfix = 2^31 - 1 (float; its row is finished by the dense path).
// Float weights only (uint8 sums are exact as accumulated and not rescored).
template <int WT>
__global__ void __launch_bounds__(256)
    k_query_prep_hybrid(const int32_t *__restrict__ qt, const void *__restrict__ qw, int32_t B, int32_t Bpad, int32_t T,
                        int32_t V, const float *__restrict__ max_abs, const int32_t *__restrict__ dup,
                        const int16_t *__restrict__ hrank, int32_t pk_shift, float *__restrict__ scale,
                        uint32_t *__restrict__ mfix, uint32_t *__restrict__ tau, uint32_t *__restrict__ cnt,
                        uint32_t *__restrict__ maxbin, int32_t *__restrict__ hshift, int8_t *__restrict__ alimb) {
    constexpr int HT = kHeavyTerms;
    __shared__ float s_hs[4][HT];
    __shared__ int32_t s_hn[4][HT], s_ha[4][HT];
    const int wv = threadIdx.x >> 6;
    const int q = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6);
    const int lane = gs_lane();
    if (q >= Bpad) return;
    for (int h = lane; h < HT; h += 64) {
        s_hs[wv][h] = 0.0f;
        s_hn[wv][h] = 0;
        s_ha[wv][h] = 0;
    }
    gs_wave_sync();
    int8_t *lim = alimb + (int64_t)q * (2 * HT);
    if (q >= B) {
        for (int h = lane; h < 2 * HT; h += 64) lim[h] = 0;
        return;
    }
    if (lane == 0) {
        tau[q] = 0;
        cnt[q] = 0;
        maxbin[q] = 0;
    }
    static_assert(WT != GS_W_U8, "float weights only");
    const int32_t *qrow = qt + (int64_t)q * T;
    const float *wrow = reinterpret_cast<const float *>(qw) + (int64_t)q * T;
    double M = 0.0, n = 0.0, At = 0.0, Ah = 0.0, Bt = 0.0, Bh = 0.0, Q = 0.0, qmax = 0.0, Wmax = 0.0, Whmax = 0.0;
    for (int j = lane; j < T; j += 64) {
        const int32_t t = qrow[j];
        if ((uint32_t)t >= (uint32_t)V) continue;
        const double m = 1.0 + (double)dup[t];
        const double aq = fabs((double)wrow[j]);
        const double W = rint(ldexp((double)max_abs[t], pk_shift));
        M += aq * (double)max_abs[t] * m;
        n += m;
        Q += aq * m;
        Wmax = fmax(Wmax, W);
        const int h = hrank[t];
        if (h >= 0) {
            Ah += aq * W * m;
            Bh += W * m;
            Whmax = fmax(Whmax, W);
            atomicAdd(&s_hs[wv][h], (float)aq);
            atomicAdd(&s_hn[wv][h], 1);
        } else {
            At += aq * W * m;
            Bt += W * m;
            qmax = fmax(qmax, aq);
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        M += __shfl_xor(M, d, 64);
        n += __shfl_xor(n, d, 64);
        At += __shfl_xor(At, d, 64);
        Ah += __shfl_xor(Ah, d, 64);
        Bt += __shfl_xor(Bt, d, 64);
        Bh += __shfl_xor(Bh, d, 64);
        Q += __shfl_xor(Q, d, 64);
        qmax = fmax(qmax, __shfl_xor(qmax, d, 64));
        Wmax = fmax(Wmax, __shfl_xor(Wmax, d, 64));
        Whmax = fmax(Whmax, __shfl_xor(Whmax, d, 64));
    }
    gs_wave_sync();
    // the largest |q| sum and occurrence count over the heavy terms; the fp32
    // sums are lifted by 1e-5 to cover their rounding (the limbs are checked
    // exactly below in any case)
    double smax = 0.0;
    int nmax = 0;
    for (int h = lane; h < HT; h += 64) {
        smax = fmax(smax, (double)s_hs[wv][h] * (1.0 + 1e-5));
        nmax = max(nmax, s_hn[wv][h]);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        smax = fmax(smax, __shfl_xor(smax, d, 64));
        nmax = max(nmax, __shfl_xor(nmax, d, 64));
    }
    M *= 1.0 + 1e-12;  // fp64 rounding of the sums themselves
    At *= 1.0 + 1e-12;
    Ah *= 1.0 + 1e-12;
    Bt *= 1.0 + 1e-12;
    Bh *= 1.0 + 1e-12;
    Q *= 1.0 + 1e-12;
    const double g64 = (2.0 * n + 2.0) * 0x1p-53 / (1.0 - (2.0 * n + 2.0) * 0x1p-53);
    const double hcap = 16383.0 - 0.5 * nmax;  // a_h <= s_h 2^(f-r) + n_h / 2 <= 16383
    const double room = 2147483646.0;
    auto r_of = [&](int f) {  // the smallest r >= 0 keeping smax 2^(f-r) <= hcap
        int r = 0;
        while (r < 40 && smax * ldexp(1.0, f - r) > hcap) ++r;
        return r;
    };
    auto fits = [&](int f, int r) {
        return (At + Ah) * ldexp(1.0, f) + 0.5 * Bt + ldexp(Bh, r - 1) < room &&
               qmax * ldexp(1.0, f) + 0.5 < 8388608.0 && r <= 30;
    };
    int f = 100;
    if (At + Ah > 0.0) f = (int)floor(log2(room / (At + Ah)));
    if (qmax > 0.0) f = min(f, (int)floor(log2(8388607.0 / qmax)));
    f = f > 100 ? 100 : (f < -100 ? -100 : f);
    int r = r_of(f);
    while (f > -100 && !fits(f, r)) r = r_of(--f);
    bool ok = hcap >= 1.0 && Wmax <= 32767.0 && Whmax <= 16383.0 && fits(f, r);
    // the heavy terms' limbs, exactly as the scorer will use them
    const float hsc = ldexpf(1.0f, f - r);
    for (int j = lane; j < T; j += 64) {
        const int32_t t = qrow[j];
        if ((uint32_t)t >= (uint32_t)V) continue;
        const int h = hrank[t];
        if (h >= 0) atomicAdd(&s_ha[wv][h], (int32_t)rintf(wrow[j] * hsc));
    }
    gs_wave_sync();
    bool out_of_range = false;
    for (int h = lane; h < HT; h += 64) {
        const int32_t av = s_ha[wv][h];
        out_of_range = out_of_range || av > 16383 || av < -16384;
    }
    ok = ok && __ballot(out_of_range) == 0;
    for (int h = lane; h < HT; h += 64) {
        const int32_t av = s_ha[wv][h];
        lim[h] = ok ? (int8_t)(av & 127) : 0;
        lim[HT + h] = ok ? (int8_t)(av >> 7) : 0;
    }
    if (lane != 0) return;
    const double Ef = 0.5 * Bt + ldexp(Bh, r - 1) + 0.5 * Q * ldexp(1.0, f);  // fixed-point units
    // + 2^kHeadShift: the slices start from the heavy-term sums rounded down to a
    // multiple of it (one-sided, k_head_scores)
    double mf = ceil(2.0 * (Ef * (1.0 + 1e-9) + g64 * M * ldexp(1.0, f + pk_shift))) + 2.0 + ldexp(1.0, kHeadShift);
    if (!ok || mf > 2147483647.0) mf = 2147483647.0;
    scale[q] = ldexpf(1.0f, f);
    mfix[q] = (uint32_t)mf;
    hshift[q] = ok ? r : 0;
}

// ---------------------------------------------------------------------- seeding

// Per query (one wave): tau from the histogram of the candidates emitted so
// far (every positive doc of the first tiles): the lower edge of the highest bin
// with at least k candidates at or above it.
__global__ void __launch_bounds__(256)
    k_tau_seed(uint32_t *__restrict__ tau, const uint32_t *__restrict__ maxbin, const uint32_t *__restrict__ hist,
               int32_t B, int32_t k) {
    const int q = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6);
    if (q >= B) return;
    raise_tau(tau + q, hist + (int64_t)q * GS_HIST_BINS, gs_load_relaxed(maxbin + q), k);
}

// ---------------------------------------------------------------------- selection

// uint8 rows: the exact top-k of the candidates is the answer.  Float rows: the
// fixed-point k-th score tau' gives the rescoring set {fixed >= tau' - mfix}.
template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_cands(const uint32_t *__restrict__ cand_doc, const uint32_t *__restrict__ cand_key,
                   const uint32_t *__restrict__ cnt, int32_t cap, int32_t k, const uint32_t *__restrict__ mfix,
                   uint32_t *__restrict__ resc_doc, uint32_t *__restrict__ resc_cnt, int32_t resc_cap,
                   const int32_t *__restrict__ perm, void *__restrict__ out_scores, int64_t *__restrict__ out_ids,
                   int32_t *__restrict__ status) {
    constexpr bool FP = WT != GS_W_U8;
    __shared__ SelStatic sst;
    SelShared sh = sel_view(sst, k);
    __shared__ uint32_t s_m;
    const int q = blockIdx.x;                 // slot
    const int row = perm ? perm[q] : q;       // query: output row
    const uint32_t n = cnt[q];
    if (n > (uint32_t)cap || n < (uint32_t)k) {
        if (threadIdx.x == 0) {
            status[row] = GS_ROW_DENSE;
            if (FP) resc_cnt[q] = 0;
        }
        return;
    }
    SrcCand32 src{cand_key + (int64_t)q * cap, cand_doc + (int64_t)q * cap, (int64_t)n};
    block_topk<32>(src, k, sh, false);
    if (!FP) {
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            reinterpret_cast<int32_t *>(out_scores)[(int64_t)row * k + i] = (int32_t)sh.key[i];
            out_ids[(int64_t)row * k + i] = (int64_t)sh.doc[i];
        }
        if (threadIdx.x == 0) status[row] = GS_ROW_DONE;
        return;
    }
    const uint32_t kth = (uint32_t)sh.key[k - 1];
    const uint32_t mf = mfix[q];
    if (kth <= mf) {  // k-th score not clear of zero by the margin
        if (threadIdx.x == 0) {
            status[row] = GS_ROW_DENSE;
            resc_cnt[q] = 0;
        }
        return;
    }
    const uint32_t t_low = kth - mf;
    if (threadIdx.x == 0) s_m = 0;
    __syncthreads();
    const uint32_t *ck = cand_key + (int64_t)q * cap;
    const uint32_t *cd = cand_doc + (int64_t)q * cap;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        if (ck[i] >= t_low) {
            const uint32_t s = atomicAdd(&s_m, 1u);
            if (s < (uint32_t)resc_cap) resc_doc[(int64_t)q * resc_cap + s] = cd[i];
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t m = s_m;
        if (m > (uint32_t)resc_cap) {
            status[row] = GS_ROW_DENSE;
            resc_cnt[q] = 0;
        } else {
            status[row] = GS_ROW_DONE;
            resc_cnt[q] = m;
        }
    }
}

// Exact fp64 score of (query, doc) candidates.  One wave per candidate: lane j
// finds query term j's posting(s) of the doc (binary search inside the doc's
// tile), then the products are summed in query-term order, which makes the sum
// bit-identical to the fp64 scatter-add.
// 1 + the index of a query's last valid term (0 when it has none): the
// rescoring loops over query terms stop there, since a batch is padded to its
// widest query (one wave, all lanes, reads the row)
__device__ __forceinline__ int valid_terms_end(const int32_t *__restrict__ qrow, int T, int V) {
    int end = 0;
    for (int j0 = 0; j0 < T; j0 += 64) {
        const int j = j0 + gs_lane();
        const uint64_t b = __ballot(j < T && (uint32_t)qrow[j] < (uint32_t)V);
        if (b) end = j0 + 64 - __clzll((long long)b);
    }
    return end;
}

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
    const int lane = gs_lane();
    const int wpb = blockDim.x >> 6;
    const int64_t row = (int64_t)n_tiles + 1;
    const store_t *wall = reinterpret_cast<const store_t *>(w);
    const int t_end = valid_terms_end(qt + (int64_t)q * T, T, V);
    for (uint32_t i = blockIdx.x * wpb + (threadIdx.x >> 6); i < m; i += gridDim.x * wpb) {
        const int32_t d = (int32_t)resc_doc[(int64_t)q * resc_cap + i];
        const int tile = d >> tile_log2;
        double s = 0.0;
        for (int j0 = 0; j0 < t_end; j0 += 64) {
            const int j = j0 + lane;
            int cnt_p = 0;       // postings of doc d in term j's list (> 1 only for duplicates)
            int64_t pos = 0;     // slot of the first of them
            double wq = 0.0;
            if (j < T) {
                const int32_t t = qt[(int64_t)q * T + j];
                if ((uint32_t)t < (uint32_t)V) {
                    const int32_t *bt = tb + (int64_t)t * row + tile;
                    int lo = bt[0];
                    const int hi = bt[1];
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
                    while (lo + cnt_p < hi && dp[lo + cnt_p] == d) ++cnt_p;
                    pos = base + lo;
                    wq = (double)qw[(int64_t)q * T + j];
                }
            }
            const double p = cnt_p ? wq * (double)gs_weight<WT>::decode(wall[pos]) : 0.0;
            // add the products in term order (ascending lanes), and duplicates in
            // list order, exactly as the scatter-add does; terms without a posting of
            // d add nothing.  Lane values are read with v_readlane (no LDS traffic).
            uint64_t hit = __ballot(cnt_p > 0);
            const uint64_t dup = __ballot(cnt_p > 1);
            while (hit) {
                const int l = __ffsll((unsigned long long)hit) - 1;
                hit &= hit - 1;
                s += gs_readlane_f64(p, l);
                if ((dup >> l) & 1ull) {
                    const int cl = __builtin_amdgcn_readlane(cnt_p, l);
                    const double wl = gs_readlane_f64(wq, l);
                    const int64_t pl = gs_readlane_i64(pos, l);
                    for (int r = 1; r < cl; ++r) s += wl * (double)gs_weight<WT>::decode(wall[pl + r]);
                }
            }
        }
        if (lane == 0) resc_key[(int64_t)q * resc_cap + i] = gs_key_f64(s);
    }
}

// The same exact fp64 score from the doc-major copy.  The wave copies the
// candidate's row (term ids and weights: one coalesced load each) into LDS, and
// lane j binary-searches query term j there instead of in term j's posting list;
// rows longer than the LDS stage are searched in place.  The row of the wave's
// next candidate is loaded into registers while the current one is searched,
// and each lane of a batch of 64 candidates looks up one candidate's row bounds.
// Rows hold a doc's postings with ascending terms and repeated (doc, term)
// entries in list order, so products and duplicates are added in the same order
// as above.
constexpr int kRescoreWaves = 4;
constexpr int kRowStage = 512;  // row entries staged in LDS per wave

// Eight workgroups (eight waves per SIMD) per CU: the waves wait on row loads, so
// more of them in flight pay for the 64-register cap (a 16-byte spill).
template <int WT>
__global__ void __launch_bounds__(64 * kRescoreWaves, 8)
    k_rescore_fwd(const int64_t *__restrict__ row_ptr, const int32_t *__restrict__ fterm,
                  const void *__restrict__ fw, int32_t V, const int32_t *__restrict__ qt,
                  const float *__restrict__ qw, int32_t T, const uint32_t *__restrict__ resc_doc,
                  const uint32_t *__restrict__ resc_cnt, int32_t resc_cap, uint64_t *__restrict__ resc_key) {
    using store_t = typename gs_weight<WT>::store_t;
    constexpr int RU = kRowStage / 64;
    __shared__ int32_t s_row[kRescoreWaves][kRowStage];
    __shared__ store_t s_rw[kRescoreWaves][kRowStage];
    __shared__ double s_prod[kRescoreWaves][64];
    const int q = blockIdx.y;
    const uint32_t m = resc_cnt[q];
    const int lane = gs_lane();
    const int w = threadIdx.x >> 6;
    int32_t *row = s_row[w];
    store_t *roww = s_rw[w];
    const store_t *wall = reinterpret_cast<const store_t *>(fw);
    const uint32_t stride = gridDim.x * kRescoreWaves;
    const int t_end = valid_terms_end(qt + (int64_t)q * T, T, V);
    // the query's first 128 terms and weights stay in registers (lane j: terms j
    // and j + 64) for all of the wave's candidates
    int32_t qt_r[2];
    double qw_r[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int j = h * 64 + lane;
        qt_r[h] = j < T ? qt[(int64_t)q * T + j] : -1;
        qw_r[h] = j < T ? (double)qw[(int64_t)q * T + j] : 0.0;
    }
    // this wave's candidates: first + c * stride, c = 0, 1, ...
    for (uint32_t first = blockIdx.x * kRescoreWaves + w; first < m; first += 64 * stride) {
        const int nc = (int)min<uint32_t>(64u, (m - first + stride - 1) / stride);
        int64_t c_r0 = 0;
        int c_n = 0;
        if (lane < nc) {
            const int32_t d = (int32_t)resc_doc[(int64_t)q * resc_cap + first + (uint32_t)lane * stride];
            c_r0 = row_ptr[d];
            c_n = (int)(row_ptr[d + 1] - c_r0);
        }
        int32_t rt[RU];
        store_t rv[RU];
        auto fetch = [&](int c) {
            const int64_t r0 = gs_readlane_i64(c_r0, c);
            const int n = __builtin_amdgcn_readlane(c_n, c);
            if (n > kRowStage) return;
#pragma unroll
            for (int u = 0; u < RU; ++u) {
                const int e = u * 64 + lane;
                rt[u] = e < n ? fterm[r0 + e] : 0;
                rv[u] = e < n ? wall[r0 + e] : store_t(0);
            }
        };
        fetch(0);
        for (int c = 0; c < nc; ++c) {
            const int64_t r0 = gs_readlane_i64(c_r0, c);
            const int n = __builtin_amdgcn_readlane(c_n, c);
            const bool staged = n <= kRowStage;
            if (staged) {
#pragma unroll
                for (int u = 0; u < RU; ++u) {
                    if (u * 64 < n) {
                        row[u * 64 + lane] = rt[u];
                        roww[u * 64 + lane] = rv[u];
                    }
                }
                gs_wave_sync();
            }
            if (c + 1 < nc) fetch(c + 1);
            auto term_at = [&](int64_t e) { return staged ? row[e] : fterm[r0 + e]; };
            auto weight_at = [&](int64_t e) { return staged ? roww[e] : wall[r0 + e]; };
            double s = 0.0;
            for (int j0 = 0; j0 < t_end; j0 += 64) {
                const int j = j0 + lane;
                int cnt_p = 0;  // entries of term j in the row (> 1 only for duplicates)
                int lo = 0;     // the first of them, within the row
                double wq = 0.0;
                if (j < T) {
                    const int32_t t = j0 == 0 ? qt_r[0] : j0 == 64 ? qt_r[1] : qt[(int64_t)q * T + j];
                    if ((uint32_t)t < (uint32_t)V) {
                        int len = n;
                        while (len > 0) {
                            const int half = len >> 1;
                            if (term_at(lo + half) < t) {
                                lo += half + 1;
                                len -= half + 1;
                            } else {
                                len = half;
                            }
                        }
                        while (lo + cnt_p < n && term_at(lo + cnt_p) == t) ++cnt_p;
                        wq = j0 == 0 ? qw_r[0] : j0 == 64 ? qw_r[1] : (double)qw[(int64_t)q * T + j];
                    }
                }
                const double p = cnt_p ? wq * (double)gs_weight<WT>::decode(weight_at(lo)) : 0.0;
                uint64_t hit = __ballot(cnt_p > 0);
                const uint64_t dup = __ballot(cnt_p > 1);
                if (!dup) {
                    // The hits' products, compacted into LDS in lane order, are
                    // added in that order by every lane: the same additions as
                    // reading them lane by lane, at one broadcast LDS read and one
                    // add per hit.
                    double *prod = s_prod[w];
                    const int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(hit >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)hit, 0u));
                    if (cnt_p > 0) prod[pos] = p;
                    gs_wave_sync();
                    const int nh = __popcll(hit);
                    for (int i = 0; i < nh; ++i) s += prod[i];
                    gs_wave_sync();  // read before the next block's products are written
                    continue;
                }
                while (hit) {
                    const int l = __ffsll((unsigned long long)hit) - 1;
                    hit &= hit - 1;
                    s += gs_readlane_f64(p, l);
                    if ((dup >> l) & 1ull) {
                        const int cl = __builtin_amdgcn_readlane(cnt_p, l);
                        const double wl = gs_readlane_f64(wq, l);
                        const int ll = __builtin_amdgcn_readlane(lo, l);
                        for (int r = 1; r < cl; ++r) s += wl * (double)gs_weight<WT>::decode(weight_at(ll + r));
                    }
                }
            }
            if (lane == 0) resc_key[(int64_t)q * resc_cap + first + (uint32_t)c * stride] = gs_key_f64(s);
            gs_wave_sync();  // the row stage is reused by the next candidate
        }
    }
}

template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_final(const uint32_t *__restrict__ resc_doc, const uint64_t *__restrict__ resc_key,
                   const uint32_t *__restrict__ resc_cnt, int32_t resc_cap, int32_t k,
                   const int32_t *__restrict__ perm, const int32_t *__restrict__ status,
                   float *__restrict__ out_scores, int64_t *__restrict__ out_ids) {
    __shared__ SelStatic sst;
    SelShared sh = sel_view(sst, k);
    const int q = blockIdx.x;            // slot
    const int row = perm ? perm[q] : q;  // query: output row
    if (status[row] != GS_ROW_DONE) return;
    SrcCand64 src{resc_key + (int64_t)q * resc_cap, resc_doc + (int64_t)q * resc_cap, (int64_t)resc_cnt[q]};
    block_topk<64>(src, k, sh, false);
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        out_scores[(int64_t)row * k + i] = (float)gs_unkey_f64(sh.key[i]);
        out_ids[(int64_t)row * k + i] = (int64_t)sh.doc[i];
    }
}

// Dense rows (fp64 or uint32) -> exact top-k.
template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_dense(const void *__restrict__ dense, int64_t ld, int64_t n_docs, int32_t k,
                   const int32_t *__restrict__ rows, int32_t r0, void *__restrict__ out_scores,
                   int64_t *__restrict__ out_ids) {
    __shared__ SelStatic sst;
    SelShared sh = sel_view(sst, k);
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

// k above kMaxK: rounds of up to kMaxK entries, each the top of the entries
// after the previous round's last one (SrcRowAfter), written one after the other.
template <int WT>
__global__ void __launch_bounds__(kSelThreads)
    k_select_dense_large(const void *__restrict__ dense, int64_t ld, int64_t n_docs, int32_t k,
                         const int32_t *__restrict__ rows, int32_t r0, void *__restrict__ out_scores,
                         int64_t *__restrict__ out_ids) {
    constexpr bool F64 = WT != GS_W_U8;
    __shared__ SelStatic sst;
    SelShared sh = sel_view(sst, kMaxK);
    const int r = blockIdx.x;
    const int q = rows ? rows[r0 + r] : r0 + r;
    const size_t esz = F64 ? sizeof(double) : sizeof(uint32_t);
    SrcRowAfter<F64> src{reinterpret_cast<const unsigned char *>(dense) + (size_t)r * (size_t)ld * esz, n_docs, 0, 0,
                         false};
    for (int done = 0; done < k;) {
        const int kr = min(kMaxK, k - done);
        const int got = block_topk<64>(src, kr, sh, true);  // == kr: k <= n_docs
        for (int i = threadIdx.x; i < got; i += blockDim.x) {
            const uint64_t key = sh.key[i] - 1;
            const int64_t o = (int64_t)q * k + done + i;
            if (F64) reinterpret_cast<float *>(out_scores)[o] = (float)gs_unkey_f64(key);
            else reinterpret_cast<int32_t *>(out_scores)[o] = (int32_t)(uint32_t)key;
            out_ids[o] = (int64_t)sh.doc[i];
        }
        if (got <= 0) break;
        src.ck = sh.key[got - 1] - 1;
        src.cd = sh.doc[got - 1];
        src.cut = true;
        done += got;
        __syncthreads();  // the next round rewrites the sort buffer
    }
}

// ---------------------------------------------------------------------- host plumbing

int dense_waves(int tile_log2, size_t acc_bytes) {
    const size_t per = (size_t(1) << tile_log2) * acc_bytes;
    int w = (int)(kTileLds / per);
    if (w > 8) w = 8;
    return w;
}

template <int WT, int UNROLL>
int launch_dense_u(DenseArgs a, int waves, size_t acc_bytes, hipStream_t s) {
    static std::atomic<bool> attr_set{false};
    auto fn = k_score_dense<WT, UNROLL>;
    const size_t lds = (size_t)waves * (size_t(1) << a.tile_log2) * acc_bytes;
    if (!attr_set.load()) {
        GS_CHECK_HIP(allow_full_lds((const void *)fn));
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

template <int WT>
int launch_dense(DenseArgs a, int waves, hipStream_t s) {
    constexpr size_t acc_bytes = WT != GS_W_U8 ? 8 : 4;
    return launch_dense_u<WT, 4>(a, waves, acc_bytes, s);
}

template <int WT, int UNROLL, bool HD>
int launch_union_hd(UnionArgs e, hipStream_t s) {
    static std::atomic<bool> attr{false};
    // scalar entry loads for groups of up to 4 slots (terms then have at most
    // 4 entries unless queries repeat terms)
    const bool se = e.G <= 4;
    auto fn = e.pk ? (se ? k_score_union<WT, UNROLL, true, true, HD> : k_score_union<WT, UNROLL, true, false, HD>)
                   : (se ? k_score_union<WT, UNROLL, false, true, HD> : k_score_union<WT, UNROLL, false, false, HD>);
    if (!attr.load()) {
        GS_CHECK_HIP(allow_full_lds((const void *)k_score_union<WT, UNROLL, true, true, HD>));
        GS_CHECK_HIP(allow_full_lds((const void *)k_score_union<WT, UNROLL, true, false, HD>));
        GS_CHECK_HIP(allow_full_lds((const void *)k_score_union<WT, UNROLL, false, true, HD>));
        GS_CHECK_HIP(allow_full_lds((const void *)k_score_union<WT, UNROLL, false, false, HD>));
        attr.store(true);
    }
    const size_t lds = ((size_t)e.G << (e.tile_log2 + 2)) + kUnionMetaLds;
    const int64_t total = (int64_t)((e.tiles + e.tiles_per_wg - 1) / e.tiles_per_wg) * e.n_groups;
    if (total == 0) return GS_OK;
    e.per_xcd = (int32_t)((total + 7) / 8);
    const int64_t grid = (int64_t)e.per_xcd * 8;
    GS_REQUIRE(grid < 0x7FFFFFFFll, "scoring grid too large (%lld workgroups)", (long long)grid);
    fn<<<(unsigned)grid, kUnionThreads, lds, s>>>(e);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

// the heavy-term start (HD) only for float weights: uint8 sums must be exact
// without rescoring
template <int WT, int UNROLL>
int launch_union(UnionArgs e, hipStream_t s) {
    if constexpr (WT != GS_W_U8)
        if (e.hsc) return launch_union_hd<WT, UNROLL, true>(e, s);
    return launch_union_hd<WT, UNROLL, false>(e, s);
}

struct SearchPlan {
    bool hyb;  // heavy terms as int8 matrix products (k_head_scores), the rest as LDS adds
    int32_t Bpad;     // slots of the heavy-term products (B rounded up to 16)
    int64_t hsc_ld;   // docs of the coarse heavy-term sums per slot: the tiles' docs rounded up to whole 512-doc blocks
    int8_t *alimb;
    int32_t *hshift;
    uint8_t *hsc;
    int S, cap, rcap, unroll, G, n_groups, ecap, gt_np, tiles_per_wg;
    int32_t *u_term, *u_ebeg, *u_count;
    uint2 *e_sw;
    float *scale;
    uint32_t *mfix, *tau, *cnt, *maxbin, *hist, *cand_doc, *cand_key, *resc_doc, *resc_cnt;
    uint64_t *resc_key;
    int32_t *perm, *qt_p;  // query order of the scoring groups and the queries in that order
    void *qw_p;
};

int check_index(const gs_index *ix) {
    GS_REQUIRE(ix, "null index");
    GS_REQUIRE(ix->wtype >= GS_W_F32 && ix->wtype <= GS_W_U8, "unknown weight type %d", ix->wtype);
    GS_REQUIRE(ix->vocab > 0 && ix->n_docs > 0 && ix->n_docs < 0x7FFFFFFFll, "bad index sizes");
    GS_REQUIRE(ix->tile_log2 >= 8 && ix->tile_log2 <= 14, "tile_log2 %d outside [8, 14]", ix->tile_log2);
    GS_REQUIRE(ix->n_tiles == (int32_t)((ix->n_docs + (1ll << ix->tile_log2) - 1) >> ix->tile_log2),
               "n_tiles %d inconsistent with n_docs and tile_log2", ix->n_tiles);
    GS_REQUIRE(ix->doc_ids_d && ix->weights_d && ix->offsets_d && ix->max_abs_d && ix->dup_d && ix->tile_bounds_d,
               "index has a null device array");
    GS_REQUIRE(!ix->fwd_ptr_d || (ix->fwd_terms_d && ix->fwd_weights_d) || ix->n_slots == 0,
               "doc-major copy without term or weight array");
    GS_REQUIRE(!ix->packed_d || ix->wtype == GS_W_U8 || (ix->packed_shift >= -200 && ix->packed_shift <= 200),
               "packed_shift %d outside [-200, 200]", ix->packed_shift);
    return GS_OK;
}

// The fused scorer reads the packed copy when it was made for this tile size and
// lies below 2^48: its per-chunk load windows carry address bits 32..47 in a
// 16-bit field (k_score_union).  Otherwise it reads the index arrays, with the
// same results.
bool packed_usable(const gs_index *ix) {
    if (!ix->packed_d || ix->packed_tile_log2 != ix->tile_log2) return false;
    const uint64_t end = (uint64_t)(uintptr_t)ix->packed_d + (uint64_t)ix->n_slots * 4u;
    return end < (1ull << 48);
}

// default tiles per scoring workgroup of a launch over `tiles` tiles
int default_tiles_per_wg(int tiles, int n_groups) {
    if ((int64_t)((tiles + 2) / 3) * n_groups >= kTripleMinWgs) return 3;
    if ((int64_t)((tiles + 1) / 2) * n_groups >= kPairMinWgs) return 2;
    return 1;
}

int next_pow2_of(int64_t n) {
    int np = 1;
    while (np < n) np <<= 1;
    return np;
}

// The hybrid search runs when the index carries the heavy terms' dense copy
// and the packed copy (integer weights), the weights are floats (uint8 sums are
// exact as accumulated and are not rescored), and the caller did not opt out.
bool hybrid_usable(const gs_index *ix, const gs_search_opts *o) {
    if (!ix->head_d || !ix->head_rank_d || !ix->heavy_d || (o && o->no_hybrid)) return false;
    return ix->wtype != GS_W_U8 && packed_usable(ix);
}

SearchPlan plan_search(const gs_index *ix, int32_t B, int32_t T, int32_t k, const gs_search_opts *o,
                       gs_arena &ar) {
    SearchPlan p;
    p.hyb = hybrid_usable(ix, o);
    // queries per group: G int32 slices of one tile fill kUnionTileLds; the group's
    // sorted term entries (next_pow2(G * T) of them) must fit the LDS sort
    int G = (int)(kUnionTileLds / 4) >> ix->tile_log2;
    if (G > 32) G = 32;
    if (G < 1) G = 1;
    if (G > B) G = B;
    auto np_of = [&](int g) { return next_pow2_of((int64_t)g * T); };
    while (G > 1 && np_of(G) > kGroupSortCap) G >>= 1;
    p.G = G;
    p.n_groups = (B + G - 1) / G;
    p.ecap = G * T;
    p.gt_np = np_of(G);
    // default first tiles scored with tau = 0: about 4 k docs, at least 4 Ki docs
    // and at most 32 Ki docs (all of their positive docs become candidates)
    const int64_t TILE = 1ll << ix->tile_log2;
    const int64_t s_min = std::max<int64_t>(1, kSeedMinDocs >> ix->tile_log2);
    const int64_t s_max = std::max<int64_t>(s_min, kSeedDocs >> ix->tile_log2);
    int64_t s_def = (4ll * k + TILE - 1) >> ix->tile_log2;
    s_def = std::min<int64_t>(std::max<int64_t>(s_def, s_min), s_max);
    // A small batch has few query groups, so all of its tiles are scored at once
    // and tau rises little after the seed: its seed is widened to about
    // kSeedFillWgs workgroups (one launch's worth), which starts tau from more docs.
    s_def = std::max<int64_t>(s_def, std::min<int64_t>(kSeedMaxTiles, (kSeedFillWgs + p.n_groups - 1) / p.n_groups));
    p.S = (o && o->sample_tiles > 0) ? o->sample_tiles : (int)s_def;
    if (p.S > ix->n_tiles) p.S = ix->n_tiles;
    if (o && o->cand_cap > 0) {
        p.cap = o->cand_cap;
    } else {
        // kCandBudget slots spread over the batch, as small batches emit more
        // candidates per query (the same reason as above); a query cannot emit
        // more candidates than there are docs
        int64_t c = std::max<int64_t>(kDefaultCandCap, std::min<int64_t>(kMaxCandCap, kCandBudget / B));
        c = std::min<int64_t>(c, (ix->n_docs + 255) / 256 * 256);
        p.cap = (int)c;
    }
    if (p.cap < 2 * k) p.cap = 2 * k;
    p.rcap = kRescoreCap;
    // default postings per lane per chunk: 16 on packed one-word postings (their
    // registers allow it), else 8
    const bool packed1 = packed_usable(ix);
    p.unroll = (o && o->unroll > 0) ? o->unroll : (packed1 ? 16 : 8);
    p.tiles_per_wg = (o && o->tiles_per_wg > 0) ? o->tiles_per_wg : 0;
    p.scale = ar.take<float>(B);
    p.mfix = ar.take<uint32_t>(B);
    p.tau = ar.take<uint32_t>(B);
    p.cnt = ar.take<uint32_t>(B);
    p.maxbin = ar.take<uint32_t>(B);
    p.resc_cnt = ar.take<uint32_t>(B);
    p.hist = ar.take<uint32_t>((size_t)B * GS_HIST_BINS);
    p.cand_doc = ar.take<uint32_t>((size_t)B * p.cap);
    p.cand_key = ar.take<uint32_t>((size_t)B * p.cap);
    p.resc_doc = ar.take<uint32_t>((size_t)B * p.rcap);
    p.resc_key = ar.take<uint64_t>((size_t)B * p.rcap);
    p.u_term = ar.take<int32_t>((size_t)p.n_groups * p.ecap);
    p.u_ebeg = ar.take<int32_t>((size_t)p.n_groups * (p.ecap + 1));
    p.u_count = ar.take<int32_t>((size_t)p.n_groups);
    p.e_sw = ar.take<uint2>((size_t)p.n_groups * p.ecap + 1);  // + 1: the scorer reads entries in pairs
    p.perm = ar.take<int32_t>((size_t)B);
    p.qt_p = ar.take<int32_t>((size_t)B * T);
    p.qw_p = ar.take<float>((size_t)B * T);  // room for fp32 or uint8 query weights
    p.Bpad = (B + 15) & ~15;
    // whole head blocks: with tiles under 512 docs an odd tile count ends half way
    // through a block, whose sums the scorer still reads
    p.hsc_ld = (((int64_t)ix->n_tiles << ix->tile_log2) + kHeadBlock - 1) / kHeadBlock * kHeadBlock;
    p.alimb = nullptr;
    p.hshift = nullptr;
    p.hsc = nullptr;
    if (p.hyb) {
        p.alimb = ar.take<int8_t>((size_t)p.Bpad * 2 * kHeavyTerms);
        p.hshift = ar.take<int32_t>((size_t)B);
        p.hsc = ar.take<uint8_t>((size_t)p.Bpad * (size_t)(p.hsc_ld / kHeadBlock) * kHscRow);
    }
    return p;
}

DenseArgs dense_args(const gs_index *ix, const int32_t *qt, const void *qw, int32_t T) {
    DenseArgs a{};
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
    SearchPlan p = plan_search(ix, B, T, k, o, ar);
    if (!ar.ok()) {
        gs_set_error("search workspace too small: need %zu bytes, got %zu", ar.used, ws_bytes);
        return GS_ENOSPC;
    }
    // optional per-phase events: start, query prep, heavy-term sums, threshold
    // seed, scoring, candidate selection, fp64 rescoring, final sort
    auto phase = [&](int i) -> int {
        if (o && o->ev_phases && o->ev_phases[i])
            GS_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(o->ev_phases[i]), s));
        return GS_OK;
    };
    int rc = phase(0);
    if (rc) return rc;
    // Scoring groups take queries that share frequent terms when the index names
    // them (heavy_d): the queries are copied in slot order and every kernel below
    // works on slots; outputs and status go to the query's own row.
    const int32_t *perm = nullptr;
    // (the hybrid scorer adds the heavy terms densely, so grouping by them saves nothing)
    if (!p.hyb && ix->heavy_d && !(o && o->batch_order) && p.G > 1 && B > p.G) {
        const int NB = p.G * (1024 / p.G);
        k_group_order<<<(B + NB - 1) / NB, 1024, 0, s>>>(qt, B, T, ix->vocab, ix->heavy_d, p.G, p.perm);
        k_permute_queries<WT><<<gs_blocks((int64_t)B * T, 256, 4096), 256, 0, s>>>(qt, qw, p.perm, B, T, p.qt_p,
                                                                                     p.qw_p);
        GS_CHECK_LAUNCH();
        perm = p.perm;
        qt = p.qt_p;
        qw = p.qw_p;
    }
    // the fused scorer reads the packed copy when it was made for this tile size
    const void *pk = packed_usable(ix) ? ix->packed_d : nullptr;
    const int32_t pkf = pk && WT != GS_W_U8 ? 1 : 0;  // integer products of the packed float weights
    if constexpr (FP) {
        if (p.hyb)
            k_query_prep_hybrid<WT><<<gs_blocks((int64_t)p.Bpad * 64, 256), 256, 0, s>>>(
                qt, qw, B, p.Bpad, T, ix->vocab, ix->max_abs_d, ix->dup_d, ix->head_rank_d, ix->packed_shift,
                p.scale, p.mfix, p.tau, p.cnt, p.maxbin, p.hshift, p.alimb);
    }
    if (!p.hyb) {
        k_query_prep<WT><<<gs_blocks((int64_t)B * 64, 256), 256, 0, s>>>(qt, qw, B, T, ix->vocab, ix->max_abs_d,
                                                                         ix->dup_d, pkf, ix->packed_shift, p.scale,
                                                                         p.mfix, p.tau, p.cnt, p.maxbin);
    }
    k_fill<uint32_t><<<gs_blocks((int64_t)B * GS_HIST_BINS, 256, 4096), 256, 0, s>>>(
        p.hist, (int64_t)B * GS_HIST_BINS, 0u);
    GS_CHECK_LAUNCH();
    {  // per group of G queries: the union of their terms (every search runs the fused scorer)
        static std::atomic<bool> attr{false};
        if (!attr.load()) {
            GS_CHECK_HIP(allow_full_lds((const void *)k_group_terms<WT>));
            attr.store(true);
        }
        k_group_terms<WT><<<p.n_groups, 1024, (size_t)p.gt_np * 12, s>>>(
            qt, qw, p.scale, pkf, B, T, ix->vocab, p.G, p.ecap, p.hyb ? ix->head_rank_d : nullptr, p.u_term,
            p.u_ebeg, p.u_count, p.e_sw);
        GS_CHECK_LAUNCH();
    }
    if ((rc = phase(1))) return rc;

    // 1. the first S tiles with tau = 0 (every positive doc is a candidate), then
    //    tau from the histogram of those candidates; 2. the remaining tiles.
    //    Both are the fused scorer: one workgroup per (run of consecutive tiles,
    //    query group) over the group's union of terms.
    UnionArgs e{};
    e.doc = ix->doc_ids_d;
    e.w = ix->weights_d;
    e.pk = pk;
    e.offsets = ix->offsets_d;
    e.tb = ix->tile_bounds_d;
    e.n_docs = ix->n_docs;
    e.V = ix->vocab;
    e.tile_log2 = ix->tile_log2;
    e.n_tiles = ix->n_tiles;
    e.B = B;
    e.G = p.G;
    e.n_groups = p.n_groups;
    e.ecap = p.ecap;
    e.u_term = p.u_term;
    e.u_ebeg = p.u_ebeg;
    e.u_count = p.u_count;
    e.e_sw = p.e_sw;
    e.tau = p.tau;
    e.cnt = p.cnt;
    e.maxbin = p.maxbin;
    e.hist = p.hist;
    e.cand_doc = p.cand_doc;
    e.cand_key = p.cand_key;
    e.mfix = p.mfix;
    e.cap = p.cap;
    e.k = k;
    auto run_union = [&](int tile_begin, int tiles) -> int {
        e.tile_begin = tile_begin;
        e.tiles = tiles;
        // Default: three tiles per workgroup when that still leaves kTripleMinWgs
        // workgroups, else two when that leaves kPairMinWgs, else one.  A further tile saves a workgroup launch
        // and the term set-up (its bounds are loaded while the previous tile is
        // scored); with few workgroups the last, partly filled round of workgroups
        // costs more.  The
        // workgroups of one tile run at the same time on one XCD and share its
        // postings in that XCD's L2; with many tiles per workgroup the groups
        // drift apart and the HBM fetch grows (~8x the index at 8 tiles).
        e.tiles_per_wg = p.tiles_per_wg > 0 ? p.tiles_per_wg : default_tiles_per_wg(tiles, p.n_groups);
        switch (p.unroll) {
            case 1: return launch_union<WT, 1>(e, s);
            case 2: return launch_union<WT, 2>(e, s);
            case 4: return launch_union<WT, 4>(e, s);
            case 16: return launch_union<WT, 16>(e, s);
            default: return launch_union<WT, 8>(e, s);
        }
    };
    if (p.hyb) {  // every slot's coarse heavy-term sums, the slices' start
        e.hsc = p.hsc;
        e.hsc_ld = p.Bpad;
        const int64_t head_rows = (ix->n_docs + kHeadBlock - 1) / kHeadBlock * kHeadBlock;
        k_head_scores<<<(unsigned)(p.hsc_ld / kHeadBlock), 512, 0, s>>>(ix->head_d, head_rows, p.alimb, p.hshift, B,
                                                                         p.Bpad, p.hsc);
        GS_CHECK_LAUNCH();
    }
    if ((rc = phase(2))) return rc;
    auto run_scorer = [&](int tile_begin, int tiles) -> int { return run_union(tile_begin, tiles); };
    e.local_k = k;  // seed launch: local k-th score thresholds (LDS-add scorer)
    if ((rc = run_scorer(0, p.S))) return rc;
    e.local_k = 0;
    k_tau_seed<<<gs_blocks((int64_t)B * 64, 256), 256, 0, s>>>(p.tau, p.maxbin, p.hist, B, k);
    GS_CHECK_LAUNCH();
    if ((rc = phase(3))) return rc;
    if (ix->n_tiles > p.S) {
        if (o && o->ev_score_begin) GS_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(o->ev_score_begin), s));
        if ((rc = run_scorer(p.S, ix->n_tiles - p.S))) return rc;
        if (o && o->ev_score_end) GS_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(o->ev_score_end), s));
    }
    if ((rc = phase(4))) return rc;

    // 3. selection (+ fp64 rescoring for float weights)
    const size_t sel_lds = sel_lds_bytes(k);
    GS_CHECK_HIP(sel_attr((const void *)k_select_cands<WT>, sel_lds));
    k_select_cands<WT><<<B, kSelThreads, sel_lds, s>>>(p.cand_doc, p.cand_key, p.cnt, p.cap, k, p.mfix, p.resc_doc,
                                                 p.resc_cnt, p.rcap, perm, out_scores, out_ids, status);
    GS_CHECK_LAUNCH();
    if ((rc = phase(5))) return rc;
    if (FP) {
        dim3 g(64u, (unsigned)B);
        // doc-major rescoring: about 16K waves over the batch (16 to 64 workgroups
        // per query), so that each wave's start-up is spread over more candidates
        // (C2: 0.51 -> 0.48 ms at 16 per query); small batches keep 64 per query
        const dim3 gf((unsigned)std::min(64, std::max(16, (16384 / kRescoreWaves) / std::max(B, 1))), (unsigned)B);
        if (ix->fwd_ptr_d)
            k_rescore_fwd<WT><<<gf, 64 * kRescoreWaves, 0, s>>>(
                ix->fwd_ptr_d, ix->fwd_terms_d, ix->fwd_weights_d, ix->vocab, qt,
                reinterpret_cast<const float *>(qw), T, p.resc_doc, p.resc_cnt, p.rcap, p.resc_key);
        else
            k_rescore<WT><<<g, 256, 0, s>>>(ix->doc_ids_d, ix->weights_d, ix->offsets_d, ix->tile_bounds_d,
                                            ix->vocab, ix->n_tiles, ix->tile_log2, qt,
                                            reinterpret_cast<const float *>(qw), T, p.resc_doc, p.resc_cnt, p.rcap,
                                            p.resc_key);
        GS_CHECK_LAUNCH();
    }
    if ((rc = phase(6))) return rc;
    if (FP) {
        GS_CHECK_HIP(sel_attr((const void *)k_select_final<WT>, sel_lds));
        k_select_final<WT><<<B, kSelThreads, sel_lds, s>>>(p.resc_doc, p.resc_key, p.resc_cnt, p.rcap, k, perm,
                                                           status, reinterpret_cast<float *>(out_scores), out_ids);
        GS_CHECK_LAUNCH();
    }
    return phase(7);
}

template <int WT>
int search_dense_impl(const gs_index *ix, const int32_t *qt, const void *qw, int32_t T, int32_t k,
                      const int32_t *rows, int32_t R, void *out_scores, int64_t *out_ids, void *ws, size_t ws_bytes,
                      hipStream_t s) {
    constexpr size_t acc_bytes = WT == GS_W_U8 ? 4 : 8;
    const int64_t TILE = 1ll << ix->tile_log2;
    const int64_t ld = (int64_t)ix->n_tiles * TILE;
    const int64_t per_row = ld * (int64_t)acc_bytes;
    const int64_t rows_per_pass = (int64_t)(ws_bytes / (size_t)per_row);
    if (rows_per_pass < 1) {
        gs_set_error("dense workspace too small: one row needs %lld bytes, got %zu", (long long)per_row, ws_bytes);
        return GS_ENOSPC;
    }
    const int waves = dense_waves(ix->tile_log2, acc_bytes);
    for (int32_t r0 = 0; r0 < R; r0 += (int32_t)rows_per_pass) {
        const int32_t n = (int32_t)std::min<int64_t>(rows_per_pass, R - r0);
        DenseArgs a = dense_args(ix, qt, qw, T);
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
        int rc = launch_dense<WT>(a, waves, s);
        if (rc) return rc;
        if (k <= kMaxK) {
            GS_CHECK_HIP(sel_attr((const void *)k_select_dense<WT>, sel_lds_bytes(k)));
            k_select_dense<WT><<<n, kSelThreads, sel_lds_bytes(k), s>>>(ws, ld, ix->n_docs, k, rows, r0,
                                                                         out_scores, out_ids);
        } else {
            GS_CHECK_HIP(sel_attr((const void *)k_select_dense_large<WT>, sel_lds_bytes(kMaxK)));
            k_select_dense_large<WT><<<n, kSelThreads, sel_lds_bytes(kMaxK), s>>>(ws, ld, ix->n_docs, k, rows, r0,
                                                                                   out_scores, out_ids);
        }
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
    GS_REQUIRE((int64_t)T <= kGroupSortCap, "query width T=%d exceeds %d terms", T, kGroupSortCap);
    gs_arena ar{nullptr, 0, 0};
    plan_search(index, B, T, k, opts, ar);
    *bytes = ar.used + 256;
    return GS_OK;
}

extern "C" int gs_search_plan(const gs_index *index, int32_t B, int32_t T, int32_t k, const gs_search_opts *opts,
                              gs_search_plan_info *out) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(B > 0 && T > 0 && k > 0 && out, "bad search sizes");
    GS_REQUIRE((int64_t)T <= kGroupSortCap, "query width T=%d exceeds %d terms", T, kGroupSortCap);
    gs_arena ar{nullptr, 0, 0};
    const SearchPlan p = plan_search(index, B, T, k, opts, ar);
    out->seed_tiles = p.S;
    out->group_size = p.G;
    out->unroll = p.unroll;
    const int rest = index->n_tiles - p.S;
    out->tiles_per_wg = p.tiles_per_wg > 0 ? p.tiles_per_wg : (rest > 0 ? default_tiles_per_wg(rest, p.n_groups) : 1);
    out->packed = packed_usable(index);
    out->hybrid = p.hyb;
    out->cand_cap = p.cap;
    return GS_OK;
}

extern "C" int gs_search_counts(const gs_index *index, int32_t B, int32_t T, int32_t k, const gs_search_opts *opts,
                                const void *workspace_d, size_t workspace_bytes, uint32_t *cand_d, uint32_t *resc_d,
                                void *stream) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(B > 0 && T > 0 && k > 0 && (int64_t)T <= kGroupSortCap, "bad search sizes");
    GS_REQUIRE(workspace_d && cand_d && resc_d, "null pointer");
    gs_arena ar{reinterpret_cast<char *>(const_cast<void *>(workspace_d)), 0, workspace_bytes};
    const SearchPlan p = plan_search(index, B, T, k, opts, ar);
    GS_REQUIRE(ar.ok(), "workspace smaller than the search's (%zu < %zu bytes)", workspace_bytes, ar.used);
    hipStream_t s = gs_stream(stream);
    GS_CHECK_HIP(hipMemcpyAsync(cand_d, p.cnt, sizeof(uint32_t) * (size_t)B, hipMemcpyDeviceToDevice, s));
    GS_CHECK_HIP(hipMemcpyAsync(resc_d, p.resc_cnt, sizeof(uint32_t) * (size_t)B, hipMemcpyDeviceToDevice, s));
    return GS_OK;
}

namespace {
int check_search_args(const gs_index *index, int32_t B, int32_t T, int32_t k, const gs_search_opts *opts,
                      const int32_t *q_terms_d, const void *q_weights_d, void *out_scores_d, int64_t *out_ids_d,
                      int32_t *status_d) {
    if (int rc = check_index(index)) return rc;
    GS_REQUIRE(B > 0 && T > 0, "empty query batch (B=%d, T=%d)", B, T);
    GS_REQUIRE(k >= 1 && k <= kMaxK && (int64_t)k <= index->n_docs, "k=%d outside [1, min(n_docs, %d)]", k, kMaxK);
    GS_REQUIRE(T <= kGroupSortCap, "query width T=%d exceeds %d terms", T, kGroupSortCap);
    GS_REQUIRE(q_terms_d && q_weights_d && out_scores_d && out_ids_d && status_d, "null pointer");
    GS_REQUIRE(!opts || (opts->tiles_per_wg >= 0 && opts->tiles_per_wg <= 64), "tiles_per_wg=%d outside [0, 64]",
               opts->tiles_per_wg);
    return GS_OK;
}

int search_dispatch(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B, int32_t T,
                    int32_t k, const gs_search_opts *opts, void *out_scores_d, int64_t *out_ids_d, int32_t *status_d,
                    void *workspace_d, size_t workspace_bytes, hipStream_t s) {
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
}  // namespace

extern "C" int gs_search(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B,
                         int32_t T, int32_t k, const gs_search_opts *opts, void *out_scores_d, int64_t *out_ids_d,
                         int32_t *status_d, void *workspace_d, size_t workspace_bytes, void *stream) {
    if (int rc = check_search_args(index, B, T, k, opts, q_terms_d, q_weights_d, out_scores_d, out_ids_d, status_d))
        return rc;
    GS_REQUIRE(workspace_d, "null workspace");
    return search_dispatch(index, q_terms_d, q_weights_d, B, T, k, opts, out_scores_d, out_ids_d, status_d,
                           workspace_d, workspace_bytes, gs_stream(stream));
}

// ---------------------------------------------------------------------- allocation-free search

// The workspace of gs_search_noalloc: a device array of the library itself, one
// per GPU the library runs on, held until the process ends.  In host code
// `scratch` is a host-side stand-in for the array, not a device address; host
// code only ever uses the address hipGetSymbolAddress reports for the current
// device (scratch_address below).
static __device__ __align__(256) unsigned char scratch[GS_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices];  // device address of `scratch` per device, set on the first call there

// Address of the current device's scratch array, looked up once per device
// with that device current.
int scratch_address(void **out) {
    int dev = -1;
    GS_CHECK_HIP(hipGetDevice(&dev));
    GS_REQUIRE(dev >= 0 && dev < kScratchDevices, "device %d outside the %d the allocation-free search serves", dev,
               kScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        GS_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        GS_REQUIRE(p != nullptr, "no device address for the scratch array on device %d", dev);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GS_OK;
}
}  // namespace

extern "C" int gs_search_noalloc(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B,
                                 int32_t T, int32_t k, const gs_search_opts *opts, void *out_scores_d,
                                 int64_t *out_ids_d, int32_t *status_d, void *stream) {
    if (int rc = check_search_args(index, B, T, k, opts, q_terms_d, q_weights_d, out_scores_d, out_ids_d, status_d))
        return rc;
    gs_arena need{nullptr, 0, 0};
    plan_search(index, B, T, k, opts, need);
    if (need.used > GS_NOALLOC_SCRATCH_BYTES) {
        gs_set_error("this search needs %zu bytes of scratch; the allocation-free search holds %zu (use fewer "
                     "queries, a smaller cand_cap, or gs_search with a workspace)",
                     need.used, (size_t)GS_NOALLOC_SCRATCH_BYTES);
        return GS_ENOSPC;
    }
    void *ws = nullptr;
    if (int rc = scratch_address(&ws)) return rc;
    return search_dispatch(index, q_terms_d, q_weights_d, B, T, k, opts, out_scores_d, out_ids_d, status_d, ws,
                           GS_NOALLOC_SCRATCH_BYTES, gs_stream(stream));
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
    GS_REQUIRE(k >= 1 && (int64_t)k <= index->n_docs, "k=%d outside [1, n_docs=%lld]", k,
               (long long)index->n_docs);
    GS_REQUIRE(q_terms_d && q_weights_d && out_scores_d && out_ids_d && workspace_d, "null pointer");
    if (R == 0) return GS_OK;
    hipStream_t s = gs_stream(stream);
    switch (index->wtype) {
        case GS_W_F32:
            return search_dense_impl<GS_W_F32>(index, q_terms_d, q_weights_d, T, k, rows_d, R, out_scores_d,
                                               out_ids_d, workspace_d, workspace_bytes, s);
        case GS_W_F16:
            return search_dense_impl<GS_W_F16>(index, q_terms_d, q_weights_d, T, k, rows_d, R, out_scores_d,
                                               out_ids_d, workspace_d, workspace_bytes, s);
        default:
            return search_dense_impl<GS_W_U8>(index, q_terms_d, q_weights_d, T, k, rows_d, R, out_scores_d,
                                              out_ids_d, workspace_d, workspace_bytes, s);
    }
}
