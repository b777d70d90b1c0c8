// Index construction and per-list checks/bounds for gfx950.
//
// The term-major layout is the reference's (lsr_benchmark_engine/
// gpusparse_retrieval.py:81-115, src/run_correctness_verification.py:32-84):
// postings of term t sit at [offsets[t], offsets[t] + lengths[t]), ascending in
// doc id (a *stable* sort of the doc-major CSR by term), padded with (-1, 0) to a
// multiple of 32 slots; offsets are the exclusive prefix sum of padded lengths.
//
// Here the transpose is a stable LSD radix sort over 8-bit digits of the term id
// (two passes for a 30522-term vocabulary).  Each pass is
//   histogram (per 4096-entry block, LDS)  ->  exclusive scan over (digit, block)
//   ->  scatter with a stable in-block rank from 64-lane ballots,
// and the last pass writes straight into the padded slot of each posting.
#include <stdarg.h>

#include <cmath>
#include <type_traits>

#include "gs_common.h"

static thread_local char g_err[512];

void gs_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" int gs_query_version(void) { return GS_ABI_VERSION; }
extern "C" int gs_heavy_term_count(void) { return kHeavyTerms; }
extern "C" const char *gs_last_error(void) { return g_err; }

namespace {

constexpr int kLdsTermsMax = 40960;  // 160 KiB of uint32 counters
constexpr int kRsThreads = 256;      // 4 waves
constexpr int kRsRounds = 16;
constexpr int kRsTile = kRsThreads * kRsRounds;  // entries per radix block
constexpr int kScanTile = 4096;

template <class T>
__global__ void k_fill(T *p, int64_t n, T v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// ------------------------------------------------------------------ block scan

// Exclusive scan across the block (blockDim multiple of 64, <= 1024).
template <class T>
__device__ T block_excl_scan(T v, T *sh /* >= 16 */, T *total) {
    const int lane = gs_lane(), wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    T x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        T o = __shfl_up(x, d, 64);
        if (lane >= d) x += o;
    }
    if (lane == 63) sh[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        T acc = 0;
        for (int w = 0; w < nw; ++w) {
            T s = sh[w];
            sh[w] = acc;
            acc += s;
        }
        sh[16] = acc;
    }
    __syncthreads();
    T r = sh[wave] + x - v;
    *total = sh[16];
    __syncthreads();
    return r;
}

// ------------------------------------------------------------------ term counts

__global__ void __launch_bounds__(1024) k_term_count_lds(const int32_t *__restrict__ idx, int64_t nnz,
                                                         int32_t V, int32_t *lengths,
                                                         unsigned long long *n_bad) {
    extern __shared__ uint32_t h[];
    for (int i = threadIdx.x; i < V; i += blockDim.x) h[i] = 0;
    __syncthreads();
    uint32_t bad = 0;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nnz;
         i += (int64_t)gridDim.x * blockDim.x) {
        int32_t t = idx[i];
        if ((uint32_t)t < (uint32_t)V)
            atomicAdd(&h[t], 1u);
        else
            ++bad;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += blockDim.x)
        if (h[i]) atomicAdd(reinterpret_cast<uint32_t *>(lengths) + i, h[i]);
    if (bad) atomicAdd(n_bad, (unsigned long long)bad);
}

__global__ void k_term_count_global(const int32_t *__restrict__ idx, int64_t nnz, int32_t V,
                                    int32_t *lengths, unsigned long long *n_bad) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nnz;
         i += (int64_t)gridDim.x * blockDim.x) {
        int32_t t = idx[i];
        if ((uint32_t)t < (uint32_t)V)
            atomicAdd(reinterpret_cast<uint32_t *>(lengths) + t, 1u);
        else
            atomicAdd(n_bad, 1ull);
    }
}

// padded = ceil32(lengths); offsets = exclusive scan(padded); optionally
// delta = offsets - exclusive scan(lengths).  Single block of 1024 threads.
__global__ void __launch_bounds__(1024) k_term_scan(const int32_t *lengths, int32_t V, int32_t *padded,
                                                    int64_t *offsets, int64_t *delta, int64_t *info,
                                                    const unsigned long long *n_bad) {
    __shared__ int64_t sh[17];
    __shared__ int64_t sh2[17];
    int64_t carry = 0, carry_seg = 0;
    for (int base = 0; base < V; base += blockDim.x) {
        int i = base + threadIdx.x;
        int64_t len = i < V ? lengths[i] : 0;
        int64_t pad = (len + 31) & ~int64_t(31);
        int64_t tot, tot2;
        int64_t ex = block_excl_scan<int64_t>(pad, sh, &tot);
        int64_t ex2 = block_excl_scan<int64_t>(len, sh2, &tot2);
        if (i < V) {
            if (padded) padded[i] = (int32_t)pad;
            if (offsets) offsets[i] = carry + ex;
            if (delta) delta[i] = (carry + ex) - (carry_seg + ex2);
        }
        carry += tot;
        carry_seg += tot2;
    }
    if (threadIdx.x == 0 && info) {
        info[0] = carry;
        info[1] = n_bad ? (int64_t)*n_bad : 0;
    }
}

// ------------------------------------------------------------------ radix sort

// Doc (row) id of every CSR entry: one wave per row.
__global__ void k_row_ids(const int64_t *__restrict__ indptr, int64_t n_rows, uint32_t *__restrict__ row_of) {
    const int lane = gs_lane();
    const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t r = wave; r < n_rows; r += nwaves) {
        int64_t b = indptr[r], e = indptr[r + 1];
        for (int64_t i = b + lane; i < e; i += 64) row_of[i] = (uint32_t)r;
    }
}

__device__ __forceinline__ uint32_t load_code(const void *p, int64_t i, int src_bytes) {
    if (src_bytes == 4) return reinterpret_cast<const uint32_t *>(p)[i];
    if (src_bytes == 2) return reinterpret_cast<const uint16_t *>(p)[i];
    return reinterpret_cast<const uint8_t *>(p)[i];
}

// Radix tile of this workgroup.  Workgroup i runs on XCD i % 8; XCD x takes the
// tiles [x*q + min(x, r), ...) in order (q, r = nblocks / 8, nblocks % 8), so the
// workgroups resident on one XCD hold neighbouring tiles, and their writes into
// one digit's region (or one digit's row of the histogram) fall next to each
// other in that XCD's L2 and leave it as whole lines.
__device__ __forceinline__ int64_t rs_tile(int64_t nblocks) {
    const int64_t p = blockIdx.x, x = p & 7;
    const int64_t q = nblocks >> 3, r = nblocks & 7;
    return x * q + (x < r ? x : r) + (p >> 3);
}

// Digit counts of one tile in LDS, kRsHistCopies copies per wave (lane l adds
// into copy l mod kRsHistCopies; the copies kRsHistStride words apart, so one
// digit's counters sit in different banks), summed at the end: a hot digit (C3's
// second pass: 46% of the term ids have high byte 0) is contended by 64 /
// kRsHistCopies lanes of a wave instead of 64 (2.7 ms with one copy per wave,
// against 1.0 ms for the evenly spread first digit).  A whole, 16-byte aligned
// tile is read as four uint4 per thread, all in flight together (the order of
// the keys does not matter).
constexpr int kRsHistCopies = 8;
constexpr int kRsHistStride = 257;
__global__ void __launch_bounds__(kRsThreads) k_rs_hist(const uint32_t *__restrict__ key, int64_t n, int shift,
                                                        uint32_t *__restrict__ hist, int64_t nblocks) {
    constexpr int kCopies = kRsThreads / 64 * kRsHistCopies;
    __shared__ uint32_t h[kCopies * kRsHistStride];
    const int tid = threadIdx.x, lane = gs_lane(), wave = tid >> 6;
    for (int i = tid; i < kCopies * kRsHistStride; i += kRsThreads) h[i] = 0;
    __syncthreads();
    const int64_t tile = rs_tile(nblocks);
    const int64_t base = tile * kRsTile;
    uint32_t *hw = h + (wave * kRsHistCopies + (lane & (kRsHistCopies - 1))) * kRsHistStride;
    if (n - base >= kRsTile && ((uintptr_t)(key + base) & 15u) == 0) {
        static_assert(kRsTile == kRsThreads * 16, "four uint4 per thread");
        const uint4 *k4 = reinterpret_cast<const uint4 *>(key + base);
        uint4 v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = k4[r * kRsThreads + tid];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            atomicAdd(&hw[(v[r].x >> shift) & 255u], 1u);
            atomicAdd(&hw[(v[r].y >> shift) & 255u], 1u);
            atomicAdd(&hw[(v[r].z >> shift) & 255u], 1u);
            atomicAdd(&hw[(v[r].w >> shift) & 255u], 1u);
        }
    } else {
        for (int r = 0; r < kRsRounds; ++r) {
            const int64_t i = base + r * kRsThreads + tid;
            if (i < n) atomicAdd(&hw[(key[i] >> shift) & 255u], 1u);
        }
    }
    __syncthreads();
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kCopies; ++w) c += h[w * kRsHistStride + tid];
    hist[(int64_t)tid * nblocks + tile] = c;
}

// Device-wide exclusive scan of uint32 (three launches).
__global__ void __launch_bounds__(1024) k_scan_reduce(const uint32_t *__restrict__ in, int64_t n,
                                                      uint32_t *__restrict__ part) {
    __shared__ uint32_t sh[17];
    const int64_t base = blockIdx.x * (int64_t)kScanTile;
    uint32_t s = 0;
    for (int j = threadIdx.x; j < kScanTile; j += blockDim.x)
        if (base + j < n) s += in[base + j];
    s = gs_wave_sum(s);
    if (gs_lane() == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += sh[w];
        part[blockIdx.x] = t;
    }
}

__global__ void __launch_bounds__(1024) k_scan_parts(uint32_t *part, int64_t nparts) {
    __shared__ uint32_t sh[17];
    uint32_t carry = 0;
    for (int64_t b = 0; b < nparts; b += blockDim.x) {
        int64_t i = b + threadIdx.x;
        uint32_t v = i < nparts ? part[i] : 0, tot;
        uint32_t ex = block_excl_scan<uint32_t>(v, sh, &tot);
        if (i < nparts) part[i] = carry + ex;
        carry += tot;
    }
}

__global__ void __launch_bounds__(1024) k_scan_down(uint32_t *__restrict__ data, int64_t n,
                                                    const uint32_t *__restrict__ part) {
    __shared__ uint32_t sh[17];
    const int64_t base = blockIdx.x * (int64_t)kScanTile;
    uint32_t carry = part[blockIdx.x];
    for (int j = 0; j < kScanTile; j += blockDim.x) {
        int64_t i = base + j + threadIdx.x;
        uint32_t v = i < n ? data[i] : 0, tot;
        uint32_t ex = block_excl_scan<uint32_t>(v, sh, &tot);
        if (i < n) data[i] = carry + ex;
        carry += tot;
    }
}

// Stable scatter of one 8-bit digit.  A block owns tile b = rs_tile(): kRsTile
// consecutive entries, wave w the kRsTile/4 of them from w*kRsTile/4 on:
//  1. every lane loads its kRsRounds entries (entry r*64 + lane of its wave's
//     range), all loads in flight together;
//  2. each wave ranks its entries among equal digits on its own, in order
//     (earlier rounds: the wave's running digit counts in LDS; earlier lanes of
//     the round: a 64-lane ballot match), with no block barrier;
//  3. the waves' digit counts give each entry its place in the block's staged
//     (digit-major, stable) order: the block's run of the digit starts at
//     l_off[digit], wave w's part of it after the parts of waves 0..w-1;
//  4. keys, then doc ids, then codes pass through one LDS buffer in staged
//     order and are written out from it: consecutive threads write consecutive
//     positions of a digit's run, so a wave's stores land in a few contiguous
//     runs instead of one scattered word per lane.  One 16 KiB buffer (not
//     three) keeps several blocks resident per CU.
// The block's run of digit t starts at global position scanned[t*nblocks + b]
// (the scanned digit-major histogram).  FINAL (the last pass of the index
// build): the entry of term k at sorted position pos goes to padded slot
// pos + delta[k], as its doc id and weight.
template <bool FINAL, int WT, bool MASK_RANK>
__global__ void __launch_bounds__(kRsThreads, 4)
    k_rs_scatter(const uint32_t *__restrict__ key_in, const uint32_t *__restrict__ doc_in,
                 const void *__restrict__ code_in, int src_code_bytes, int64_t n, int shift, int bits,
                 const uint32_t *__restrict__ scanned, int64_t nblocks, uint32_t *__restrict__ key_out,
                 uint32_t *__restrict__ doc_out, uint32_t *__restrict__ code_out,
                 const int64_t *__restrict__ delta, int32_t *__restrict__ final_doc,
                 void *__restrict__ final_w) {
    constexpr int kWaves = kRsThreads / 64, kPerWave = kRsTile / kWaves;
    __shared__ uint32_t s_buf[kRsTile];
    __shared__ uint32_t g_run[256];          // global position of this block's run of each digit
    __shared__ uint32_t l_off[256];          // start of each digit's run in the staged order
    __shared__ uint32_t wcnt[kWaves][256];   // per wave: digits seen, then the wave's offset in the run
    __shared__ uint64_t peers_of[kWaves][256];  // per wave: the lanes of a round holding each digit
    __shared__ uint32_t sh[17];
    const int tid = threadIdx.x, wave = tid >> 6, lane = gs_lane();
    const int64_t tile = rs_tile(nblocks);
    const int64_t base = tile * kRsTile;
    const int cnt = (int)(n - base < kRsTile ? n - base : kRsTile);
    const int wbase = wave * kPerWave;

    uint32_t k[kRsRounds], d[kRsRounds], c[kRsRounds], lp[kRsRounds];
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r) {
        const int j = wbase + r * 64 + lane;
        k[r] = d[r] = 0;
        if (j < cnt) {
            k[r] = key_in[base + j];
            d[r] = doc_in[base + j];
        }
    }
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        wcnt[w][tid] = 0;
        peers_of[w][tid] = 0;
    }
    {
        const int64_t idx = (int64_t)tid * nblocks + tile;
        g_run[tid] = scanned[idx];
    }
    __syncthreads();
    // 2. wave-local stable ranks (lp = rank among the wave's entries of that
    // digit): the running count of the digit in the wave plus the lane's rank
    // among the round's lanes holding it.  MASK_RANK: those lanes are found by
    // ORing their bits into the digit's mask in LDS -- for digits that rarely
    // repeat within a round (the index build's first pass: consecutive CSR
    // entries are different terms); else by matching the digit's bits across the
    // wave with ballots, for digits a round shares (a term id's top byte, 46% of
    // C3's postings have high byte 0; a sorted list's doc-id bytes above the
    // lowest), whose lanes would serialize on one LDS atomic: C3's index build
    // 6.72 -> 6.54 ms with the mask in its first pass, the doc-major copy's
    // passes 8.3 -> 9.0 ms with it.  Keys are below 2^(shift + bits).
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r) {
        const bool valid = wbase + r * 64 + lane < cnt;
        const uint32_t dig = (k[r] >> shift) & 255u;
        uint64_t peers = 0;
        uint32_t seen = 0;
        if (!MASK_RANK) {
            peers = __ballot(valid);
            for (int b = 0; b < bits; ++b) {
                const bool bit = (dig >> b) & 1u;
                const uint64_t m = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            if (valid) seen = wcnt[wave][dig];
        } else {
            if (valid) atomicOr(&peers_of[wave][dig], 1ull << lane);
            gs_wave_sync();
            if (valid) {
                peers = peers_of[wave][dig];
                seen = wcnt[wave][dig];
            }
        }
        gs_wave_sync();
        const uint32_t rank =
            __builtin_amdgcn_mbcnt_hi((uint32_t)(peers >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)peers, 0u));
        lp[r] = seen + rank;
        if (valid && rank == 0) {
            wcnt[wave][dig] = seen + (uint32_t)__popcll(peers);
            if (MASK_RANK) peers_of[wave][dig] = 0;
        }
        gs_wave_sync();
    }
    __syncthreads();
    // 3. the block's digit counts, their exclusive scan, and each wave's offset in a run
    {
        uint32_t tot_d = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t x = wcnt[w][tid];
            wcnt[w][tid] = tot_d;
            tot_d += x;
        }
        uint32_t tot;
        l_off[tid] = block_excl_scan<uint32_t>(tot_d, sh, &tot);
    }
    __syncthreads();  // every digit's l_off is read by other waves below
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r) {
        const uint32_t dig = (k[r] >> shift) & 255u;
        lp[r] += l_off[dig] + wcnt[wave][dig];
    }
    // 4. keys, then doc ids, then codes through the staging buffer
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r)
        if (wbase + r * 64 + lane < cnt) s_buf[lp[r]] = k[r];
    // the codes are loaded only now, into the registers the keys held
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r) {
        const int j = wbase + r * 64 + lane;
        c[r] = j < cnt ? load_code(code_in, base + j, src_code_bytes) : 0u;
    }
    __syncthreads();
    // destination of staged entry i*256 + tid: sorted position, or padded slot (FINAL)
    using Dst = typename std::conditional<FINAL, int64_t, uint32_t>::type;
    Dst dst[kRsRounds];
#pragma unroll
    for (int i = 0; i < kRsRounds; ++i) {
        const int j = i * kRsThreads + tid;
        dst[i] = 0;
        if (j < cnt) {
            const uint32_t kk = s_buf[j];
            const uint32_t dig = (kk >> shift) & 255u;
            const uint32_t pos = g_run[dig] + ((uint32_t)j - l_off[dig]);
            if (FINAL) {
                dst[i] = (int64_t)pos + delta[kk];
            } else {
                dst[i] = pos;
                key_out[pos] = kk;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r)
        if (wbase + r * 64 + lane < cnt) s_buf[lp[r]] = d[r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRsRounds; ++i) {
        const uint32_t v = s_buf[i * kRsThreads + tid];
        if (i * kRsThreads + tid < cnt) {
            if (FINAL)
                final_doc[dst[i]] = (int32_t)v;
            else
                doc_out[dst[i]] = v;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRsRounds; ++r)
        if (wbase + r * 64 + lane < cnt) s_buf[lp[r]] = c[r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRsRounds; ++i) {
        const uint32_t v = s_buf[i * kRsThreads + tid];
        if (i * kRsThreads + tid < cnt) {
            if (!FINAL) {  // the next pass reads the codes at their own width
                if (WT == GS_W_F32)
                    code_out[dst[i]] = v;
                else if (WT == GS_W_F16)
                    reinterpret_cast<uint16_t *>(code_out)[dst[i]] = (uint16_t)v;
                else
                    reinterpret_cast<uint8_t *>(code_out)[dst[i]] = (uint8_t)v;
            } else if (WT == GS_W_F32)
                reinterpret_cast<uint32_t *>(final_w)[dst[i]] = v;
            else if (WT == GS_W_F16)
                reinterpret_cast<uint16_t *>(final_w)[dst[i]] = (uint16_t)v;
            else
                reinterpret_cast<uint8_t *>(final_w)[dst[i]] = (uint8_t)v;
        }
    }
}

// ------------------------------------------------------------------ forward (doc-major) copy

// Exclusive scan of the list lengths (int64), single block; excl[V] = total.
__global__ void __launch_bounds__(1024) k_len_scan(const int32_t *lengths, int32_t V, int64_t *excl) {
    __shared__ int64_t sh[17];
    int64_t carry = 0;
    for (int base = 0; base < V; base += blockDim.x) {
        const int i = base + threadIdx.x;
        const int64_t len = i < V ? lengths[i] : 0;
        int64_t tot;
        const int64_t ex = block_excl_scan<int64_t>(len, sh, &tot);
        if (i < V) excl[i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) excl[V] = carry;
}

// The postings of the term-major index without padding, in list order: key =
// doc id (n_docs for ids outside [0, n_docs), which then sort after every row),
// payload = term id and weight bits.  Each wave takes a segment of 64 * kFlatRounds
// consecutive flattened postings, whatever the list lengths: lane 0 finds the
// segment's first term by binary search over the exclusive scan `excl`, then
// every lane walks forward to the term of its posting.
constexpr int kFlatRounds = 16;
__global__ void k_flatten(const int32_t *__restrict__ doc_ids, const void *__restrict__ w, int w_bytes,
                          const int64_t *__restrict__ offsets, int32_t V, int64_t n_docs,
                          const int64_t *__restrict__ excl, int64_t nnz, uint32_t *__restrict__ key,
                          uint32_t *__restrict__ term, uint32_t *__restrict__ code) {
    const int lane = gs_lane();
    const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    constexpr int64_t SEG = 64 * kFlatRounds;
    for (int64_t s0 = wave * SEG; s0 < nnz; s0 += nwaves * SEG) {
        // last t with excl[t] <= s0 (excl is non-decreasing, excl[0] = 0, excl[V] = nnz > s0)
        int lo = 0, hi = V;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (excl[mid] <= s0) lo = mid;
            else hi = mid;
        }
        int t = lo;
        for (int r = 0; r < kFlatRounds; ++r) {
            const int64_t i = s0 + r * 64 + lane;
            if (i >= nnz) break;
            while (excl[t + 1] <= i) ++t;  // t < V: excl[V] = nnz > i
            const int64_t src = offsets[t] + (i - excl[t]);
            const int32_t d = doc_ids[src];
            key[i] = (d >= 0 && d < n_docs) ? (uint32_t)d : (uint32_t)n_docs;
            term[i] = (uint32_t)t;
            code[i] = load_code(w, src, w_bytes);
        }
    }
}

// Sorted (doc, term, weight) entries -> row pointers, term ids and typed weights.
template <int WT>
__global__ void k_unpack_rows(const uint32_t *__restrict__ doc, const uint32_t *__restrict__ term,
                              const uint32_t *__restrict__ code, int64_t n, int64_t n_docs,
                              int64_t *__restrict__ row_ptr, int32_t *__restrict__ fwd_term, void *__restrict__ fwd_w) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i <= n; i += (int64_t)gridDim.x * blockDim.x) {
        // rows (prev, cur] start at i: the first entry of a doc, or the end for the
        // trailing docs (keys are <= n_docs, the key n_docs marks ids out of range)
        const int64_t prev = i > 0 ? (int64_t)doc[i - 1] : -1;
        const int64_t cur = i < n ? (int64_t)doc[i] : n_docs;
        for (int64_t d = prev + 1; d <= cur; ++d) row_ptr[d] = i;
        if (i < n) {
            fwd_term[i] = (int32_t)term[i];
            if (WT == GS_W_F32) reinterpret_cast<uint32_t *>(fwd_w)[i] = code[i];
            else if (WT == GS_W_F16) reinterpret_cast<uint16_t *>(fwd_w)[i] = (uint16_t)code[i];
            else reinterpret_cast<uint8_t *>(fwd_w)[i] = (uint8_t)code[i];
        }
    }
}

// Padding slots [offsets + lengths, offsets + padded) <- (-1, 0).
template <int WT>
__global__ void k_fill_pads(const int64_t *__restrict__ offsets, const int32_t *__restrict__ lengths,
                            const int32_t *__restrict__ padded, int32_t V, int32_t *__restrict__ doc_ids,
                            void *__restrict__ w) {
    const int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t t = g >> 5;
    const int j = (int)(g & 31);
    if (t >= V) return;
    const int64_t slot = offsets[t] + lengths[t] + j;
    if (slot >= offsets[t] + padded[t]) return;
    doc_ids[slot] = -1;
    if (WT == GS_W_F32)
        reinterpret_cast<float *>(w)[slot] = 0.0f;
    else if (WT == GS_W_F16)
        reinterpret_cast<uint16_t *>(w)[slot] = 0;
    else
        reinterpret_cast<uint8_t *>(w)[slot] = 0;
}

// ------------------------------------------------------------------ per-list scans

constexpr int kListParts = 16;  // waves per list for the per-list passes
constexpr int kListUnroll = 8;  // loads in flight per lane in those passes

template <int WT>
__device__ __forceinline__ float weight_as_float(const void *w, int64_t i) {
    if (WT == GS_W_F32) return reinterpret_cast<const float *>(w)[i];
    if (WT == GS_W_F16) return (float)reinterpret_cast<const _Float16 *>(w)[i];
    return (float)reinterpret_cast<const uint8_t *>(w)[i];
}

// max and max |w| per list, as monotone keys (max_key) and abs bits (max_abs_bits).
template <int WT>
__global__ void k_list_max(const void *__restrict__ w, const int64_t *__restrict__ offsets,
                           const int32_t *__restrict__ lengths, int32_t V, uint32_t *max_key,
                           uint32_t *max_abs_bits) {
    const int lane = gs_lane();
    const int64_t wv = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t t = wv / kListParts;
    const int part = (int)(wv % kListParts);
    if (t >= V) return;
    const int64_t L = lengths[t], o = offsets[t];
    const int64_t per = (L + kListParts - 1) / kListParts;
    const int64_t b = part * per, e = b + per < L ? b + per : L;
    if (b >= e) return;
    uint32_t mk = 0, ma = 0;
    // kListUnroll loads in flight per lane (a long list's parts are latency-bound)
    for (int64_t i0 = b + lane; i0 < e; i0 += 64 * kListUnroll) {
        float v[kListUnroll];
#pragma unroll
        for (int u = 0; u < kListUnroll; ++u) {
            const int64_t i = i0 + 64 * u;
            v[u] = i < e ? weight_as_float<WT>(w, o + i) : weight_as_float<WT>(w, o + b);
        }
#pragma unroll
        for (int u = 0; u < kListUnroll; ++u) {
            const uint32_t k = gs_key_f32(v[u]), a = __float_as_uint(fabsf(v[u]));
            mk = k > mk ? k : mk;
            ma = a > ma ? a : ma;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        uint32_t o1 = __shfl_xor(mk, d, 64), o2 = __shfl_xor(ma, d, 64);
        mk = o1 > mk ? o1 : mk;
        ma = o2 > ma ? o2 : ma;
    }
    if (lane == 0) {
        atomicMax(max_key + t, mk);
        atomicMax(max_abs_bits + t, ma);
    }
}

__global__ void k_list_max_final(const uint32_t *max_key, const uint32_t *max_abs_bits,
                                 const int32_t *lengths, int32_t V, float *max_scores, float *max_abs) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= V) return;
    const bool nz = lengths[t] > 0;
    if (max_scores) max_scores[t] = nz ? gs_unkey_f32(max_key[t]) : 0.0f;
    if (max_abs) max_abs[t] = nz ? __uint_as_float(max_abs_bits[t]) : 0.0f;
}

// Non-ascending flag and count of equal neighbours per list.
__global__ void k_check_lists(const int32_t *__restrict__ doc, const int64_t *__restrict__ offsets,
                              const int32_t *__restrict__ lengths, int32_t V, int32_t *bad, int32_t *dup) {
    const int lane = gs_lane();
    const int64_t wv = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t t = wv / kListParts;
    const int part = (int)(wv % kListParts);
    if (t >= V) return;
    const int64_t L = lengths[t], o = offsets[t];
    const int64_t per = (L + kListParts - 1) / kListParts;
    int64_t b = part * per;
    const int64_t e = b + per < L ? b + per : L;
    if (b < 1) b = 1;
    if (b >= e) return;
    uint32_t nbad = 0, ndup = 0;
    for (int64_t i0 = b + lane; i0 < e; i0 += 64 * kListUnroll) {
        int32_t cur[kListUnroll], prev[kListUnroll];
#pragma unroll
        for (int u = 0; u < kListUnroll; ++u) {
            const int64_t i = i0 + 64 * u < e ? i0 + 64 * u : b;  // past the end: a pair counted below as neither
            cur[u] = doc[o + i];
            prev[u] = doc[o + i - 1];
        }
#pragma unroll
        for (int u = 0; u < kListUnroll; ++u) {
            const bool in = i0 + 64 * u < e;
            nbad += in && cur[u] < prev[u];
            ndup += in && cur[u] == prev[u];
        }
    }
    nbad = gs_wave_sum(nbad);
    ndup = gs_wave_sum(ndup);
    if (lane == 0) {
        if (nbad) atomicOr(reinterpret_cast<uint32_t *>(bad) + t, 1u);
        if (ndup) atomicAdd(reinterpret_cast<uint32_t *>(dup) + t, ndup);
    }
}

__global__ void __launch_bounds__(1024) k_count_flags(const int32_t *flags, int32_t V, int64_t *out) {
    __shared__ uint32_t sh[17];
    uint32_t c = 0;
    for (int i = threadIdx.x; i < V; i += blockDim.x) c += flags[i] != 0;
    c = gs_wave_sum(c);
    if (gs_lane() == 0) sh[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += sh[w];
        out[0] = t;
    }
}

__device__ __forceinline__ int64_t lower_bound_i32(const int32_t *a, int64_t n, int64_t x) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        int64_t mid = (lo + hi) >> 1;
        if ((int64_t)a[mid] < x)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

__global__ void k_chunk_bounds(const int32_t *__restrict__ doc, const int64_t *__restrict__ offsets,
                               const int32_t *__restrict__ lengths, int32_t V, int64_t n_docs,
                               int64_t chunk, int64_t n_chunks, int64_t *__restrict__ bounds) {
    const int64_t total = (n_chunks + 1) * (int64_t)V;
    for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < total;
         g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t c = g / V, t = g % V;
        const int64_t edge = c < n_chunks ? c * chunk : n_docs;
        const int64_t o = offsets[t];
        bounds[g] = o + lower_bound_i32(doc + o, lengths[t], edge);
    }
}

__global__ void k_tile_bounds(const int32_t *__restrict__ doc, const int64_t *__restrict__ offsets,
                              const int32_t *__restrict__ lengths, int32_t V, int32_t tile_log2,
                              int64_t n_tiles, int32_t *__restrict__ bounds) {
    const int64_t row = n_tiles + 1;
    const int64_t total = row * (int64_t)V;
    for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < total;
         g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = g / row, j = g % row;
        const int64_t o = offsets[t];
        bounds[g] = (int32_t)lower_bound_i32(doc + o, lengths[t], j << tile_log2);
    }
}

// Packed scoring copy of the postings for one tile size, one 32-bit word per
// slot: the byte offset of its doc's word in a tile slice, (doc mod tile) * 4 <
// 2^16, in the low 16 bits and the weight above it -- the uint8 weight, or for
// float weights the int16 rint(w * 2^shift) (w * 2^shift is exact in fp64 and
// rounded once, half to even; clamped to +-32767).  Padding slots (doc < 0) hold 0.
template <int WT>
__device__ __forceinline__ uint32_t pack_word_of(int32_t d, typename gs_weight<WT>::store_t wv, uint32_t mask,
                                                 int32_t shift) {
    if (d < 0) return 0u;
    const uint32_t off = ((uint32_t)d & mask) << 2;
    uint32_t wq;
    if (WT == GS_W_U8) {
        wq = (uint32_t)wv;
    } else {
        const double r = rint(ldexp((double)gs_weight<WT>::decode(wv), shift));
        const int32_t q = (int32_t)fmin(fmax(r, -32767.0), 32767.0);
        wq = (uint32_t)(uint16_t)(int16_t)q;
    }
    return off | (wq << 16);
}

template <int WT>
__device__ __forceinline__ uint32_t pack_word(int32_t d, const void *__restrict__ w, int64_t i, uint32_t mask,
                                              int32_t shift) {
    if (d < 0) return 0u;
    return pack_word_of<WT>(d, reinterpret_cast<const typename gs_weight<WT>::store_t *>(w)[i], mask, shift);
}

// VEC: four consecutive slots per thread and iteration (16-byte doc and word
// accesses, one load of four weights; the arrays aligned to that), the last
// n % 4 slots one by one.  Packing four at a time cut C3's packed-copy build
// from 9.5 to 8.55 ms.
template <int WT, bool VEC>
__global__ void k_pack_postings(const int32_t *__restrict__ doc, const void *__restrict__ w, int64_t n,
                                int32_t tile_log2, int32_t shift, uint32_t *__restrict__ out) {
    const uint32_t mask = (1u << tile_log2) - 1u;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t done = 0;
    if constexpr (VEC) {
        using store_t = typename gs_weight<WT>::store_t;
        typedef store_t w4_t __attribute__((ext_vector_type(4)));
        const int64_t n4 = n >> 2;
        for (int64_t i = t; i < n4; i += stride) {
            const int4 d = reinterpret_cast<const int4 *>(doc)[i];
            const w4_t v = reinterpret_cast<const w4_t *>(w)[i];
            reinterpret_cast<uint4 *>(out)[i] =
                make_uint4(pack_word_of<WT>(d.x, v.x, mask, shift), pack_word_of<WT>(d.y, v.y, mask, shift),
                           pack_word_of<WT>(d.z, v.z, mask, shift), pack_word_of<WT>(d.w, v.w, mask, shift));
        }
        done = n4 << 2;
    }
    for (int64_t i = done + t; i < n; i += stride) out[i] = pack_word<WT>(doc[i], w, i, mask, shift);
}

// Bank-aware order of the packed copy inside each (term, tile) sub-range.  The
// scorer adds a sub-range's postings 64 at a time -- one ds_add_u32 per lane,
// groups aligned to the sub-range's start -- into the words of their docs, and
// postings whose docs agree mod 64 fall in one LDS bank.  Any order inside a
// sub-range gives the same sums.  The sub-range is cut into blocks of
// kArrangeBlock = 1024 postings from its start, and each block of n > 64
// postings (G groups, the last one holding n_last = n - 64 (G - 1)) is
// rewritten "column-major by residue": its postings sorted by (doc mod 64, doc)
// are dealt to the groups in turn -- the k-th of them to group k mod G, position
// k / G, while every group has room at that position (k < n_last * G), then to
// the first G - 1 groups only.  The postings of one residue land in different
// groups while they last, so a group holds a residue ceil(count / G) times at
// most (2 for random docs), where docs in ascending order pile 3-5 lanes onto
// one bank.
// One wave per kArrangeTiles tiles of one term (lane j < kArrangeTiles holds
// tile j's sub-range); the wave takes the blocks of its sub-ranges one after the
// other, in place in the packed copy that k_pack_postings has written in slot
// order: every lane loads its words of the block (all loads in flight; a word's
// offset bits give its doc's residue: (doc mod tile) mod 64, the scorer's bank,
// which orders a sub-range's docs as doc mod 64 does), the residues are counted
// in LDS, each posting is ranked among its residue (the lanes of its 64-posting
// group with that residue OR their bits into an LDS mask; its rank is the count
// of lower lanes in it, after the running count of the residue), its word goes
// to its place in an LDS copy of the block, and the wave writes the copy back.
// Dealing whole sub-ranges (up to 16384 postings at 16384-doc tiles) instead of
// blocks puts each 64-posting group's words on 64 different cache lines: those
// stores took 5.3 of that kernel's 7.4 ms at C3 (tile 14), where the blocked
// pass takes 2.1 ms (4.5 ms reading the doc ids and weights instead of the
// packed words), with the same scorer times.
constexpr int kArrangeGroups = 16;                  // 64-posting groups per block
constexpr int kArrangeBlock = 64 * kArrangeGroups;  // postings per block
constexpr int kArrangeTiles = 8;                    // tiles of one term per wave

__global__ void __launch_bounds__(256)
    k_pack_arrange(const int64_t *__restrict__ offsets, const int32_t *__restrict__ tb, int32_t V, int64_t n_tiles,
                   uint32_t *__restrict__ out) {
    __shared__ uint32_t s_cnt[4][64], s_run[4][64];
    __shared__ uint64_t s_peers[4][64];
    __shared__ uint32_t s_block[4][kArrangeBlock];
    const int lane = gs_lane(), wave = threadIdx.x >> 6;
    const int64_t per_term = (n_tiles + kArrangeTiles - 1) / kArrangeTiles;  // waves per term
    const int64_t gw = blockIdx.x * 4ll + wave;                               // this wave
    s_peers[wave][lane] = 0;
    int64_t s = 0;
    int n = 0;
    if (gw < (int64_t)V * per_term && lane < kArrangeTiles) {
        const int64_t t = gw / per_term, j = (gw - t * per_term) * kArrangeTiles + lane;
        if (j < n_tiles) {
            const int32_t *b = tb + t * (n_tiles + 1) + j;
            n = b[1] - b[0];
            s = offsets[t] + b[0];
        }
    }
    uint64_t todo = __ballot(n > 64);
    while (todo) {
        const int src = __ffsll((long long)todo) - 1;
        todo &= todo - 1;
        const int64_t ss = ((int64_t)__builtin_amdgcn_readlane((int)(s >> 32), src) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)s, src);
        const int nn = __builtin_amdgcn_readlane(n, src);
        for (int b0 = 0; nn - b0 > 64; b0 += kArrangeBlock) {  // the blocks of more than 64 postings
            const int nb = min(kArrangeBlock, nn - b0);
            uint32_t *blk = out + ss + b0;
            const int G = (nb + 63) >> 6, nl = nb - 64 * (G - 1);
            // quotients below 1024 from a float reciprocal: within one, corrected below
            const float rcp_g = 1.0f / (float)G, rcp_g1 = 1.0f / (float)(G - 1);
            uint32_t wd[kArrangeGroups];
#pragma unroll
            for (int u = 0; u < kArrangeGroups; ++u) {
                const int i = u * 64 + lane;
                wd[u] = i < nb ? blk[i] : 0u;
            }
            s_cnt[wave][lane] = 0;
            gs_wave_sync();
#pragma unroll
            for (int u = 0; u < kArrangeGroups; ++u)
                if (u * 64 + lane < nb) atomicAdd(&s_cnt[wave][(wd[u] >> 2) & 63u], 1u);
            gs_wave_sync();
            const uint32_t cnt = s_cnt[wave][lane];
            uint32_t x = cnt;  // inclusive scan of the residue counts over the lanes
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = __shfl_up(x, d, 64);
                if (lane >= d) x += o;
            }
            s_run[wave][lane] = x - cnt;  // next place of residue `lane` in (residue, doc) order
            gs_wave_sync();
#pragma unroll
            for (int u = 0; u < kArrangeGroups; ++u) {
                if (u >= G) continue;  // uniform: the block's groups only
                const bool valid = u * 64 + lane < nb;
                const uint32_t r = (wd[u] >> 2) & 63u;
                if (valid) atomicOr(&s_peers[wave][r], 1ull << lane);
                gs_wave_sync();
                uint64_t peers = 0;
                uint32_t seen = 0;
                if (valid) {
                    peers = s_peers[wave][r];
                    seen = s_run[wave][r];
                }
                gs_wave_sync();
                const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(peers >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)peers, 0u));
                if (valid && rank == 0) {  // the residue's first lane advances its place and clears its mask
                    s_run[wave][r] = seen + (uint32_t)__popcll(peers);
                    s_peers[wave][r] = 0;
                }
                if (valid) {
                    // k < nb: group and position, k divided by G (k < nl G) or, past that, k - nl G by G - 1
                    const uint32_t k = seen + rank;
                    const bool all = k < (uint32_t)(nl * G);
                    const uint32_t num = all ? k : k - (uint32_t)(nl * G);
                    const uint32_t den = all ? (uint32_t)G : (uint32_t)(G - 1);
                    uint32_t q = (uint32_t)((float)num * (all ? rcp_g : rcp_g1));
                    const int32_t rem = (int32_t)(num - q * den);
                    q = rem < 0 ? q - 1u : (rem >= (int32_t)den ? q + 1u : q);
                    const uint32_t grp = num - q * den, pos = all ? q : (uint32_t)nl + q;
                    s_block[wave][grp * 64 + pos] = wd[u];
                }
                gs_wave_sync();
            }
#pragma unroll
            for (int u = 0; u < kArrangeGroups; ++u) {
                const int i = u * 64 + lane;
                if (i < nb) blk[i] = s_block[wave][i];
            }
            gs_wave_sync();  // the next block reuses the LDS copy and counts
        }
    }
}

// Block-wide exclusive prefix sum over 1024 threads (one value each); returns
// the thread's offset and writes the total to *total.  Uses sh[16].
__device__ uint32_t block_excl_scan_1024(uint32_t v, uint32_t *sh, uint32_t *total) {
    const int lane = gs_lane(), wave = threadIdx.x >> 6;
    const uint32_t inc = gs_wave_incl_scan(v);
    if (lane == 63) sh[wave] = inc;
    __syncthreads();
    uint32_t base = 0, tot = 0;
    for (int w = 0; w < 16; ++w) {
        const uint32_t x = sh[w];
        base += w < wave ? x : 0u;
        tot += x;
    }
    __syncthreads();
    *total = tot;
    return base + inc - v;
}

// The kHeavyTerms non-empty lists with the most postings, by (length
// descending, term ascending), -1 past the number of non-empty lists.  One
// workgroup of 1024 threads: an 8-bit-per-pass radix select finds the
// kHeavyTerms-th largest length L; the lists longer than L and the first lists
// (by term id) of length L are collected, then sorted by one wave.
__global__ void __launch_bounds__(1024) k_heavy_terms(const int32_t *__restrict__ len, int32_t V,
                                                      int32_t *__restrict__ heavy) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sh[16];
    __shared__ uint32_t s_pref, s_need;
    __shared__ int32_t s_sel[kHeavyTerms];
    const int tid = threadIdx.x, lane = gs_lane();
    const int per = (V + 1023) / 1024;
    const int t0 = tid * per, t1 = min(V, t0 + per);
    // non-empty lists
    uint32_t nz = 0;
    for (int t = t0; t < t1; ++t) nz += len[t] > 0;
    uint32_t n_nz;
    block_excl_scan_1024(nz, sh, &n_nz);
    // L = the kHeavyTerms-th largest length (1 when there are fewer non-empty lists)
    uint32_t L = 1;
    if (n_nz > (uint32_t)kHeavyTerms) {
        if (tid == 0) {
            s_pref = 0;
            s_need = kHeavyTerms;
        }
        uint32_t mask = 0;
        for (int shift = 24; shift >= 0; shift -= 8) {
            if (tid < 256) hist[tid] = 0;
            __syncthreads();
            const uint32_t pref = s_pref;
            for (int t = t0; t < t1; ++t) {
                const uint32_t v = (uint32_t)max(len[t], 0);
                if (v && (v & mask) == pref) atomicAdd(&hist[(v >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid < 64) {  // lane l holds digits 255 - 4l .. 252 - 4l, highest first
                uint32_t c[4], sum = 0;
                for (int j = 0; j < 4; ++j) sum += (c[j] = hist[255 - 4 * lane - j]);
                const uint32_t inc = gs_wave_incl_scan(sum);
                const uint32_t need = s_need;
                const uint64_t hit = __ballot(inc >= need);
                const int l = __ffsll((unsigned long long)hit) - 1;  // exists: the prefix holds >= need values
                if (lane == l) {
                    uint32_t cum = inc - sum;
                    int j = 0;
                    while (cum + c[j] < need) cum += c[j++];
                    s_pref = pref | ((uint32_t)(255 - 4 * lane - j) << shift);
                    s_need = need - cum;
                }
            }
            mask |= 255u << shift;
            __syncthreads();
        }
        L = s_pref;
    }
    // collect the lists longer than L, then the first `need` lists of length L
    uint32_t gt = 0, eq = 0;
    for (int t = t0; t < t1; ++t) {
        const uint32_t v = (uint32_t)max(len[t], 0);
        gt += v > L;
        eq += v == L;
    }
    uint32_t n_gt, n_eq;
    uint32_t o_gt = block_excl_scan_1024(gt, sh, &n_gt);
    uint32_t o_eq = block_excl_scan_1024(eq, sh, &n_eq);
    const uint32_t need_eq = min(n_eq, (uint32_t)kHeavyTerms - min(n_gt, (uint32_t)kHeavyTerms));
    if (tid < kHeavyTerms) s_sel[tid] = -1;
    __syncthreads();
    for (int t = t0; t < t1; ++t) {
        const uint32_t v = (uint32_t)max(len[t], 0);
        if (v > L && o_gt < (uint32_t)kHeavyTerms) s_sel[o_gt++] = t;
        if (v == L) {
            if (o_eq < need_eq) s_sel[n_gt + o_eq] = t;
            ++o_eq;
        }
    }
    __syncthreads();
    // bitonic sort of the picks by (length desc, term asc), -1 last: key =
    // length << 32 | (2^31 - 1 - term), 0 for no pick, sorted descending
    __shared__ uint64_t s_key[kHeavyTerms];
    if (tid < kHeavyTerms) {
        const int32_t t = s_sel[tid];
        s_key[tid] = t < 0 ? 0ull : ((uint64_t)(uint32_t)len[t] << 32) | (uint32_t)(0x7FFFFFFF - t);
    }
    for (int size = 2; size <= kHeavyTerms; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            const int j = tid ^ stride;
            if (tid < kHeavyTerms && j > tid) {
                const uint64_t x = s_key[tid], y = s_key[j];
                if (((tid & size) == 0) ? x < y : x > y) {
                    s_key[tid] = y;
                    s_key[j] = x;
                }
            }
        }
    __syncthreads();
    (void)lane;
    if (tid < kHeavyTerms) {
        const uint64_t key = s_key[tid];
        heavy[tid] = key ? (int32_t)(0x7FFFFFFF - (uint32_t)key) : -1;
    }
}

// Dense copy of the heavy terms' packed integer weights, an operand of the
// hybrid search's int8 matrix products: row d holds two limb vectors of
// kHeavyTerms bytes, low = wq & 127 and high = wq >> 7 (arithmetic), for wq the
// packed copy's integer weight of (d, heavy[h]) (pack_word_of) and 0 where doc d
// lacks term h.  Every |wq| <= 16383 fits: low in [0, 127], high in [-128, 127].
// One workgroup per kHeadFillBlocks consecutive blocks of kHeadFillDocs docs,
// taken one after the other: per heavy term, a lane finds the term's postings
// of the block (they start where the previous block's ended; their end is
// searched within the block's width, which bounds it when the list holds each
// doc at most once, and over the rest of the list otherwise), the waves write
// their limbs into the block's rows staged in LDS (kHeadStrideWords words apart,
// an odd number, so lanes on consecutive docs write distinct banks), and the
// workgroup writes the rows out whole (a byte scatter straight into the rows
// would cost a write transaction per byte), clearing the stage behind it.  The
// block's postings of all heavy terms are taken as one flat range (an exclusive
// scan of the per-term counts; a thread finds its posting's term by binary search
// of it), kHeadFillUnroll per thread with their loads in flight together.
// Rows past n_docs stay zero.  One block per workgroup with two full binary
// searches per term and 128-byte rows in LDS (a 32-way bank conflict on every
// byte write) took 2.25 ms at C3.
constexpr int kHeadRow = 2 * kHeavyTerms;            // bytes per row
constexpr int kHeadRowWords = kHeadRow / 4;
constexpr int kHeadStrideWords = kHeadRowWords + 1;  // LDS row stride, odd
constexpr int kHeadFillDocs = 32768 / kHeadRow;      // docs per block: 256 for 64 heavy terms
constexpr int kHeadFillBlocks = 4;                   // blocks per workgroup
constexpr int kHeadFillUnroll = 8;                   // postings per thread loaded together
static_assert(kHeadFillDocs % 16 == 0 && kHeavyTerms <= 256, "head fill block shape");

// the first position in doc[lo, hi) (ascending) holding a doc >= d
__device__ __forceinline__ int64_t lower_doc(const int32_t *__restrict__ doc, int64_t lo, int64_t hi, int64_t d) {
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)doc[mid] < d) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

template <int WT>
__global__ void __launch_bounds__(256)
    k_head_fill(const int32_t *__restrict__ doc, const void *__restrict__ w, const int64_t *__restrict__ offsets,
                const int32_t *__restrict__ lengths, const int32_t *__restrict__ heavy, int32_t shift, int64_t n_docs,
                int64_t n_rows, int8_t *__restrict__ head) {
    __shared__ uint32_t stage[kHeadFillDocs * kHeadStrideWords];
    __shared__ int64_t s_lo[kHeavyTerms], s_hi[kHeavyTerms];
    __shared__ uint32_t s_pre[kHeavyTerms], s_total;
    const int tid = threadIdx.x, lane = gs_lane(), wave = tid >> 6;
    int8_t *stage8 = reinterpret_cast<int8_t *>(stage);
    for (int i = tid; i < kHeadFillDocs * kHeadStrideWords; i += blockDim.x) stage[i] = 0u;
    // thread h < kHeavyTerms follows heavy term h: [lo, e) its postings from the block on
    int32_t t = -1;
    int64_t lo = 0, e = 0;
    if (tid < kHeavyTerms) {
        t = heavy[tid];
        if (t >= 0) {
            lo = offsets[t];
            e = lo + lengths[t];
        }
    }
    const auto *wall = reinterpret_cast<const typename gs_weight<WT>::store_t *>(w);
    const int64_t first = (int64_t)blockIdx.x * (kHeadFillBlocks * kHeadFillDocs);
    for (int k = 0; k < kHeadFillBlocks; ++k) {
        const int64_t d0 = first + (int64_t)k * kHeadFillDocs;
        if (d0 >= n_rows) break;
        const int64_t d1 = min(d0 + kHeadFillDocs, n_docs);
        if (tid < kHeavyTerms) {
            int64_t hi = lo;
            if (t >= 0 && d0 < d1) {
                if (k == 0) lo = lower_doc(doc, lo, e, d0);
                const int64_t cap = min(e, lo + (d1 - d0));
                hi = lower_doc(doc, lo, cap, d1);
                if (hi == cap && cap < e && (int64_t)doc[cap] < d1) hi = lower_doc(doc, cap, e, d1);  // repeated docs
            }
            s_lo[tid] = lo;
            s_hi[tid] = hi;
            lo = hi;
        }
        __syncthreads();
        // the block's postings of all heavy terms in one flat range: term h's at
        // [s_pre[h], s_pre[h] + s_hi[h] - s_lo[h])
        if (wave == 0) {
            uint32_t carry = 0;
            for (int c = 0; c < kHeavyTerms; c += 64) {
                const uint32_t v = (uint32_t)(s_hi[c + lane] - s_lo[c + lane]);
                const uint32_t inc = gs_wave_incl_scan(v);
                s_pre[c + lane] = carry + inc - v;
                carry += __shfl(inc, 63, 64);
            }
            if (lane == 0) s_total = carry;
        }
        __syncthreads();
        const uint32_t total = s_total;
        for (uint32_t f0 = 0; f0 < total; f0 += 256u * kHeadFillUnroll) {
            int32_t dv[kHeadFillUnroll], hv[kHeadFillUnroll];
            typename gs_weight<WT>::store_t wv[kHeadFillUnroll];
#pragma unroll
            for (int u = 0; u < kHeadFillUnroll; ++u) {  // every load in flight before any is used
                const uint32_t f = f0 + (uint32_t)(u * 256 + tid);
                hv[u] = -1;
                if (f < total) {
                    int h = 0;  // the last term whose range starts at or before f (a non-empty one)
#pragma unroll
                    for (int step = kHeavyTerms / 2; step > 0; step >>= 1)
                        if (s_pre[h + step] <= f) h += step;
                    const int64_t i = s_lo[h] + (int64_t)(f - s_pre[h]);
                    hv[u] = h;
                    dv[u] = doc[i];  // in [d0, d1): the range above
                    wv[u] = wall[i];
                }
            }
#pragma unroll
            for (int u = 0; u < kHeadFillUnroll; ++u) {
                const int h = hv[u];
                if (h >= 0) {
                    // the packed word's weight half: uint8 0..255, or int16 rint(w 2^shift)
                    const int32_t wq = (int32_t)(int16_t)(pack_word_of<WT>(dv[u], wv[u], 0u, shift) >> 16);
                    int8_t *row = stage8 + (int64_t)(dv[u] - d0) * (4 * kHeadStrideWords);
                    row[h] = (int8_t)(wq & 127);
                    row[kHeavyTerms + h] = (int8_t)(wq >> 7);
                }
            }
        }
        __syncthreads();
        const int rows = (int)min<int64_t>(kHeadFillDocs, n_rows - d0);
        uint32_t *out = reinterpret_cast<uint32_t *>(head + d0 * kHeadRow);
        for (int i = tid; i < rows * kHeadRowWords; i += blockDim.x) {
            const int r = i / kHeadRowWords, a = r * kHeadStrideWords + (i - r * kHeadRowWords);
            out[i] = stage[a];
            stage[a] = 0u;
        }
        __syncthreads();
    }
}

// rank[t] = h for t = heavy[h], -1 for every other term
__global__ void k_head_rank(int32_t V, int16_t *__restrict__ rank) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < V; i += (int64_t)gridDim.x * blockDim.x)
        rank[i] = -1;
}
__global__ void k_head_rank_set(const int32_t *__restrict__ heavy, int32_t V, int16_t *__restrict__ rank) {
    const int h = threadIdx.x;
    if (h < kHeavyTerms) {
        const int32_t t = heavy[h];
        if (t >= 0 && t < V) rank[t] = (int16_t)h;
    }
}

}  // namespace

// ====================================================================== C ABI

extern "C" int gs_index_count(const int32_t *indices_d, int64_t nnz, int32_t vocab, int32_t *lengths_d,
                              int32_t *padded_d, int64_t *offsets_d, int64_t *info_d, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(nnz >= 0 && nnz < 0xFFFFFFFFll, "nnz %lld outside [0, 2^32-1)", (long long)nnz);
    GS_REQUIRE(lengths_d && padded_d && offsets_d && info_d, "null output pointer");
    GS_REQUIRE(nnz == 0 || indices_d, "null indices");
    hipStream_t s = gs_stream(stream);
    // info_d doubles as the 64-bit bad-entry counter until the scan writes it.
    unsigned long long *n_bad = reinterpret_cast<unsigned long long *>(info_d + 1);
    k_fill<int32_t><<<gs_blocks(vocab, 256), 256, 0, s>>>(lengths_d, vocab, 0);
    k_fill<int64_t><<<1, 64, 0, s>>>(info_d, 2, 0);
    GS_CHECK_LAUNCH();
    if (nnz > 0) {
        if (vocab <= kLdsTermsMax) {
            size_t lds = sizeof(uint32_t) * (size_t)vocab;
            GS_CHECK_HIP(hipFuncSetAttribute((const void *)k_term_count_lds,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            unsigned blocks = gs_blocks(nnz, 1024 * 64, 512);
            k_term_count_lds<<<blocks, 1024, lds, s>>>(indices_d, nnz, vocab, lengths_d, n_bad);
        } else {
            k_term_count_global<<<gs_blocks(nnz, 256, 65536), 256, 0, s>>>(indices_d, nnz, vocab,
                                                                          lengths_d, n_bad);
        }
        GS_CHECK_LAUNCH();
    }
    k_term_scan<<<1, 1024, 0, s>>>(lengths_d, vocab, padded_d, offsets_d, nullptr, info_d, n_bad);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

namespace {
struct FillPlan {
    int passes;
    int64_t nblocks;
    int64_t hist_n;
    int64_t nparts;
};
FillPlan fill_plan(int64_t nnz, int32_t vocab) {
    FillPlan p;
    int bits = 0;
    while (bits < 31 && (1ll << bits) < (int64_t)vocab) ++bits;
    p.passes = bits <= 8 ? 1 : (bits + 7) / 8;
    p.nblocks = (nnz + kRsTile - 1) / kRsTile;
    if (p.nblocks < 1) p.nblocks = 1;
    p.hist_n = 256 * p.nblocks;
    p.nparts = (p.hist_n + kScanTile - 1) / kScanTile;
    return p;
}
size_t fill_layout(int64_t nnz, int32_t vocab, gs_arena &a, uint32_t **row_of, uint32_t *kb[2],
                   uint32_t *db[2], uint32_t *cb[2], uint32_t **hist, uint32_t **parts, int64_t **delta,
                   uint32_t **mk, uint32_t **ma) {
    FillPlan p = fill_plan(nnz, vocab);
    *row_of = a.take<uint32_t>(nnz);
    int nbuf = p.passes >= 3 ? 2 : (p.passes == 2 ? 1 : 0);
    for (int b = 0; b < 2; ++b) {
        kb[b] = b < nbuf ? a.take<uint32_t>(nnz) : nullptr;
        db[b] = b < nbuf ? a.take<uint32_t>(nnz) : nullptr;
        cb[b] = b < nbuf ? a.take<uint32_t>(nnz) : nullptr;
    }
    *hist = a.take<uint32_t>(p.hist_n);
    *parts = a.take<uint32_t>(p.nparts);
    *delta = a.take<int64_t>(vocab);
    *mk = a.take<uint32_t>(vocab);
    *ma = a.take<uint32_t>(vocab);
    return a.used;
}
}  // namespace

extern "C" size_t gs_index_fill_workspace(int64_t nnz, int32_t vocab) {
    gs_arena a{nullptr, 0, 0};
    uint32_t *r, *kb[2], *db[2], *cb[2], *h, *pp, *mk, *ma;
    int64_t *dl;
    return fill_layout(nnz, vocab, a, &r, kb, db, cb, &h, &pp, &dl, &mk, &ma) + 256;
}

template <int WT>
static int index_fill_impl(const int64_t *indptr_d, const int32_t *indices_d, const void *data_d,
                           int64_t n_docs, int64_t nnz, int32_t vocab, const int64_t *offsets_d,
                           const int32_t *lengths_d, const int32_t *padded_d, int32_t *doc_ids_d,
                           void *weights_d, float *max_scores_d, float *max_abs_d, void *ws,
                           size_t ws_bytes, hipStream_t s) {
    gs_arena a{reinterpret_cast<char *>(ws), 0, ws_bytes};
    uint32_t *row_of, *kb[2], *db[2], *cb[2], *hist, *parts, *mk, *ma;
    int64_t *delta;
    fill_layout(nnz, vocab, a, &row_of, kb, db, cb, &hist, &parts, &delta, &mk, &ma);
    if (!a.ok()) {
        gs_set_error("index_fill workspace too small: need %zu bytes, got %zu", a.used, ws_bytes);
        return GS_ENOSPC;
    }
    const FillPlan p = fill_plan(nnz, vocab);
    const int src_bytes = WT == GS_W_F32 ? 4 : (WT == GS_W_F16 ? 2 : 1);

    // per-term delta = offsets - exclusive scan(lengths): padded slot of a sorted position
    k_term_scan<<<1, 1024, 0, s>>>(lengths_d, vocab, nullptr, nullptr, delta, nullptr, nullptr);
    k_fill_pads<WT><<<gs_blocks((int64_t)vocab * 32, 256), 256, 0, s>>>(offsets_d, lengths_d, padded_d,
                                                                        vocab, doc_ids_d, weights_d);
    GS_CHECK_LAUNCH();
    if (nnz > 0) {
        k_row_ids<<<gs_blocks(n_docs * 64, 256, 65536), 256, 0, s>>>(indptr_d, n_docs, row_of);
        GS_CHECK_LAUNCH();
        const uint32_t *key_in = reinterpret_cast<const uint32_t *>(indices_d);
        const uint32_t *doc_in = row_of;
        const void *code_in = data_d;
        int code_bytes = src_bytes;
        int cur = 0;
        for (int pass = 0; pass < p.passes; ++pass) {
            const int shift = 8 * pass;
            const bool last = pass == p.passes - 1;
            int bits = 8;
            {
                int total_bits = 0;
                while (total_bits < 31 && (1ll << total_bits) < (int64_t)vocab) ++total_bits;
                if (total_bits < 1) total_bits = 1;
                int rem = total_bits - shift;
                bits = rem < 8 ? rem : 8;
                if (bits < 1) bits = 1;
            }
            k_rs_hist<<<(unsigned)p.nblocks, kRsThreads, 0, s>>>(key_in, nnz, shift, hist, p.nblocks);
            k_scan_reduce<<<(unsigned)p.nparts, 1024, 0, s>>>(hist, p.hist_n, parts);
            k_scan_parts<<<1, 1024, 0, s>>>(parts, p.nparts);
            k_scan_down<<<(unsigned)p.nparts, 1024, 0, s>>>(hist, p.hist_n, parts);
            GS_CHECK_LAUNCH();
            if (last) {
                k_rs_scatter<true, WT, false><<<(unsigned)p.nblocks, kRsThreads, 0, s>>>(
                    key_in, doc_in, code_in, code_bytes, nnz, shift, bits, hist, p.nblocks, nullptr, nullptr,
                    nullptr, delta, doc_ids_d, weights_d);
            } else {
                // the lowest digit of the term ids of a CSR's consecutive entries rarely repeats
                auto scatter = pass == 0 ? k_rs_scatter<false, WT, true> : k_rs_scatter<false, WT, false>;
                scatter<<<(unsigned)p.nblocks, kRsThreads, 0, s>>>(key_in, doc_in, code_in, code_bytes, nnz, shift,
                                                                   bits, hist, p.nblocks, kb[cur], db[cur], cb[cur],
                                                                   nullptr, nullptr, nullptr);
                key_in = kb[cur];
                doc_in = db[cur];
                code_in = cb[cur];
                cur ^= 1;
            }
            GS_CHECK_LAUNCH();
        }
    }
    // max_scores / max_abs
    k_fill<uint32_t><<<gs_blocks(vocab, 256), 256, 0, s>>>(mk, vocab, 0u);
    k_fill<uint32_t><<<gs_blocks(vocab, 256), 256, 0, s>>>(ma, vocab, 0u);
    k_list_max<WT><<<gs_blocks((int64_t)vocab * kListParts * 64, 256), 256, 0, s>>>(
        weights_d, offsets_d, lengths_d, vocab, mk, ma);
    k_list_max_final<<<gs_blocks(vocab, 256), 256, 0, s>>>(mk, ma, lengths_d, vocab, max_scores_d,
                                                          max_abs_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_index_fill(const int64_t *indptr_d, const int32_t *indices_d, const void *data_d,
                             int32_t wtype, int64_t n_docs, int64_t nnz, int32_t vocab,
                             const int64_t *offsets_d, const int32_t *lengths_d, const int32_t *padded_d,
                             int64_t n_slots, int32_t *doc_ids_d, void *weights_d, float *max_scores_d,
                             float *max_abs_d, void *workspace_d, size_t workspace_bytes, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(n_docs >= 0 && n_docs < 0x7FFFFFFFll, "n_docs %lld outside [0, 2^31-1)", (long long)n_docs);
    GS_REQUIRE(nnz >= 0 && nnz < 0xFFFFFFFFll, "nnz %lld outside [0, 2^32-1)", (long long)nnz);
    GS_REQUIRE(n_slots >= nnz, "n_slots %lld < nnz %lld", (long long)n_slots, (long long)nnz);
    GS_REQUIRE(indptr_d && offsets_d && lengths_d && padded_d, "null input pointer");
    GS_REQUIRE(nnz == 0 || (indices_d && data_d), "null CSR arrays");
    GS_REQUIRE(n_slots == 0 || (doc_ids_d && weights_d), "null output arrays");
    hipStream_t s = gs_stream(stream);
    switch (wtype) {
        case GS_W_F32:
            return index_fill_impl<GS_W_F32>(indptr_d, indices_d, data_d, n_docs, nnz, vocab, offsets_d,
                                             lengths_d, padded_d, doc_ids_d, weights_d, max_scores_d,
                                             max_abs_d, workspace_d, workspace_bytes, s);
        case GS_W_F16:
            return index_fill_impl<GS_W_F16>(indptr_d, indices_d, data_d, n_docs, nnz, vocab, offsets_d,
                                             lengths_d, padded_d, doc_ids_d, weights_d, max_scores_d,
                                             max_abs_d, workspace_d, workspace_bytes, s);
        case GS_W_U8:
            return index_fill_impl<GS_W_U8>(indptr_d, indices_d, data_d, n_docs, nnz, vocab, offsets_d,
                                            lengths_d, padded_d, doc_ids_d, weights_d, max_scores_d,
                                            max_abs_d, workspace_d, workspace_bytes, s);
        default:
            gs_set_error("unknown weight type %d", wtype);
            return GS_EINVAL;
    }
}

extern "C" int gs_check_lists(const int32_t *doc_ids_d, const int64_t *offsets_d, const int32_t *lengths_d,
                              int32_t vocab, int32_t *bad_d, int32_t *dup_d, int64_t *info_d, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(offsets_d && lengths_d && bad_d && dup_d && info_d, "null pointer");
    hipStream_t s = gs_stream(stream);
    k_fill<int32_t><<<gs_blocks(vocab, 256), 256, 0, s>>>(bad_d, vocab, 0);
    k_fill<int32_t><<<gs_blocks(vocab, 256), 256, 0, s>>>(dup_d, vocab, 0);
    k_check_lists<<<gs_blocks((int64_t)vocab * kListParts * 64, 256), 256, 0, s>>>(
        doc_ids_d, offsets_d, lengths_d, vocab, bad_d, dup_d);
    k_count_flags<<<1, 1024, 0, s>>>(bad_d, vocab, info_d);
    k_count_flags<<<1, 1024, 0, s>>>(lengths_d, vocab, info_d + 1);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_list_max(const void *weights_d, int32_t wtype, const int64_t *offsets_d, const int32_t *lengths_d,
                           int32_t vocab, float *max_scores_d, float *max_abs_d, void *workspace_d,
                           size_t workspace_bytes, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(weights_d && offsets_d && lengths_d && workspace_d, "null pointer");
    GS_REQUIRE(workspace_bytes >= 2 * sizeof(uint32_t) * (size_t)vocab, "list_max workspace too small");
    hipStream_t s = gs_stream(stream);
    uint32_t *mk = reinterpret_cast<uint32_t *>(workspace_d), *ma = mk + vocab;
    k_fill<uint32_t><<<gs_blocks(2 * (int64_t)vocab, 256), 256, 0, s>>>(mk, 2 * (int64_t)vocab, 0u);
    const unsigned g = gs_blocks((int64_t)vocab * kListParts * 64, 256);
    switch (wtype) {
        case GS_W_F32: k_list_max<GS_W_F32><<<g, 256, 0, s>>>(weights_d, offsets_d, lengths_d, vocab, mk, ma); break;
        case GS_W_F16: k_list_max<GS_W_F16><<<g, 256, 0, s>>>(weights_d, offsets_d, lengths_d, vocab, mk, ma); break;
        case GS_W_U8: k_list_max<GS_W_U8><<<g, 256, 0, s>>>(weights_d, offsets_d, lengths_d, vocab, mk, ma); break;
        default: gs_set_error("unknown weight type %d", wtype); return GS_EINVAL;
    }
    k_list_max_final<<<gs_blocks(vocab, 256), 256, 0, s>>>(mk, ma, lengths_d, vocab, max_scores_d, max_abs_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_chunk_bounds(const int32_t *doc_ids_d, const int64_t *offsets_d, const int32_t *lengths_d,
                               int32_t vocab, int64_t n_docs, int64_t doc_chunk, int64_t *bounds_d,
                               void *stream) {
    GS_REQUIRE(vocab > 0 && n_docs >= 0, "bad sizes");
    GS_REQUIRE(doc_chunk > 0, "doc_chunk must be positive, got %lld", (long long)doc_chunk);
    const int64_t n_chunks = (n_docs + doc_chunk - 1) / doc_chunk;
    const int64_t total = (n_chunks + 1) * (int64_t)vocab;
    k_chunk_bounds<<<gs_blocks(total, 256, 1 << 16), 256, 0, gs_stream(stream)>>>(
        doc_ids_d, offsets_d, lengths_d, vocab, n_docs, doc_chunk, n_chunks, bounds_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_tile_bounds(const int32_t *doc_ids_d, const int64_t *offsets_d, const int32_t *lengths_d,
                              int32_t vocab, int64_t n_docs, int32_t tile_log2, int32_t *bounds_d,
                              void *stream) {
    GS_REQUIRE(vocab > 0 && n_docs >= 0, "bad sizes");
    GS_REQUIRE(tile_log2 >= 6 && tile_log2 <= 16, "tile_log2 %d outside [6, 16]", tile_log2);
    const int64_t n_tiles = (n_docs + (1ll << tile_log2) - 1) >> tile_log2;
    const int64_t total = (n_tiles + 1) * (int64_t)vocab;
    k_tile_bounds<<<gs_blocks(total, 256, 1 << 16), 256, 0, gs_stream(stream)>>>(
        doc_ids_d, offsets_d, lengths_d, vocab, tile_log2, n_tiles, bounds_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

// ------------------------------------------------------------------ forward copy ABI

namespace {
struct FwdLayout {
    int64_t *excl;
    uint32_t *kb[2], *tb[2], *cb[2], *hist, *parts;
};
size_t fwd_layout(int64_t nnz, int32_t vocab, gs_arena &a, FwdLayout &l) {
    const FillPlan p = fill_plan(nnz, vocab);
    l.excl = a.take<int64_t>((size_t)vocab + 1);
    for (int b = 0; b < 2; ++b) {
        l.kb[b] = a.take<uint32_t>(nnz);
        l.tb[b] = a.take<uint32_t>(nnz);
        l.cb[b] = a.take<uint32_t>(nnz);
    }
    l.hist = a.take<uint32_t>(p.hist_n);
    l.parts = a.take<uint32_t>(p.nparts);
    return a.used;
}
// One wave per CSR row: sets *unsorted when a column index is smaller than the
// one before it in the same row (equal neighbours, a repeated term, are sorted).
__global__ void __launch_bounds__(256) k_rows_sorted(const int64_t *__restrict__ indptr,
                                                     const int32_t *__restrict__ indices, int64_t n_rows,
                                                     int32_t *__restrict__ unsorted) {
    const int lane = gs_lane();
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
    bool bad = false;
    for (int64_t r = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6; r < n_rows; r += waves) {
        const int64_t b = indptr[r], e = indptr[r + 1];
        for (int64_t i = b + 1 + lane; i < e; i += 64) bad |= indices[i] < indices[i - 1];
    }
    if (__ballot(bad) && lane == 0) atomicOr(reinterpret_cast<unsigned int *>(unsorted), 1u);
}

}  // namespace

extern "C" size_t gs_forward_fill_workspace(int64_t nnz, int32_t vocab) {
    gs_arena a{nullptr, 0, 0};
    FwdLayout l;
    return fwd_layout(nnz, vocab, a, l) + 256;
}

// ------------------------------------------------------------------ CSR row order

extern "C" int gs_rows_sorted(const int64_t *indptr_d, const int32_t *indices_d, int64_t n_rows,
                              int32_t *unsorted_d, void *stream) {
    GS_REQUIRE(n_rows >= 0, "n_rows %lld is negative", (long long)n_rows);
    GS_REQUIRE(unsorted_d && (n_rows == 0 || (indptr_d && indices_d)), "null pointer");
    hipStream_t s = gs_stream(stream);
    k_fill<int32_t><<<1, 64, 0, s>>>(unsorted_d, 1, 0);
    if (n_rows > 0)
        k_rows_sorted<<<gs_blocks(n_rows * 64, 256, 1 << 16), 256, 0, s>>>(indptr_d, indices_d, n_rows, unsorted_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_forward_fill(const int32_t *doc_ids_d, const void *weights_d, int32_t wtype,
                               const int64_t *offsets_d, const int32_t *lengths_d, int32_t vocab, int64_t n_docs,
                               int64_t nnz, int64_t *row_ptr_d, int32_t *fwd_terms_d, void *fwd_weights_d,
                               void *workspace_d, size_t workspace_bytes, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(n_docs > 0 && n_docs < 0x7FFFFFFFll, "n_docs %lld outside [1, 2^31-1)", (long long)n_docs);
    GS_REQUIRE(nnz >= 0 && nnz < 0xFFFFFFFFll, "nnz %lld outside [0, 2^32-1)", (long long)nnz);
    GS_REQUIRE(wtype >= GS_W_F32 && wtype <= GS_W_U8, "unknown weight type %d", wtype);
    GS_REQUIRE(doc_ids_d && weights_d && offsets_d && lengths_d && row_ptr_d && workspace_d, "null pointer");
    GS_REQUIRE(nnz == 0 || (fwd_terms_d && fwd_weights_d), "null output arrays");
    hipStream_t s = gs_stream(stream);
    gs_arena a{reinterpret_cast<char *>(workspace_d), 0, workspace_bytes};
    FwdLayout l;
    fwd_layout(nnz, vocab, a, l);
    if (!a.ok()) {
        gs_set_error("forward_fill workspace too small: need %zu bytes, got %zu", a.used, workspace_bytes);
        return GS_ENOSPC;
    }
    const int w_bytes = wtype == GS_W_F32 ? 4 : (wtype == GS_W_F16 ? 2 : 1);
    k_len_scan<<<1, 1024, 0, s>>>(lengths_d, vocab, l.excl);
    GS_CHECK_LAUNCH();
    int cur = 0;
    if (nnz > 0) {
        k_flatten<<<gs_blocks((nnz + 63) / 64 * 64 / kFlatRounds + 64, 256, 65536), 256, 0, s>>>(
            doc_ids_d, weights_d, w_bytes, offsets_d, vocab, n_docs, l.excl, nnz, l.kb[0], l.tb[0], l.cb[0]);
        GS_CHECK_LAUNCH();
        // stable LSD radix sort by doc id: rows come out with ascending terms, and
        // the entries of a repeated (doc, term) pair keep their list order
        const FillPlan p = fill_plan(nnz, vocab);
        int total_bits = 1;  // keys are <= n_docs
        while (total_bits < 31 && (1ll << total_bits) <= n_docs) ++total_bits;
        for (int shift = 0; shift < total_bits; shift += 8) {
            const int bits = total_bits - shift < 8 ? total_bits - shift : 8;
            k_rs_hist<<<(unsigned)p.nblocks, kRsThreads, 0, s>>>(l.kb[cur], nnz, shift, l.hist, p.nblocks);
            k_scan_reduce<<<(unsigned)p.nparts, 1024, 0, s>>>(l.hist, p.hist_n, l.parts);
            k_scan_parts<<<1, 1024, 0, s>>>(l.parts, p.nparts);
            k_scan_down<<<(unsigned)p.nparts, 1024, 0, s>>>(l.hist, p.hist_n, l.parts);
            k_rs_scatter<false, GS_W_F32, false><<<(unsigned)p.nblocks, kRsThreads, 0, s>>>(
                l.kb[cur], l.tb[cur], l.cb[cur], 4, nnz, shift, bits, l.hist, p.nblocks, l.kb[cur ^ 1],
                l.tb[cur ^ 1], l.cb[cur ^ 1], nullptr, nullptr, nullptr);
            GS_CHECK_LAUNCH();
            cur ^= 1;
        }
    }
    const unsigned g = gs_blocks(nnz + 1, 256, 1 << 16);
    switch (wtype) {
        case GS_W_F32:
            k_unpack_rows<GS_W_F32><<<g, 256, 0, s>>>(l.kb[cur], l.tb[cur], l.cb[cur], nnz, n_docs, row_ptr_d,
                                                      fwd_terms_d, fwd_weights_d);
            break;
        case GS_W_F16:
            k_unpack_rows<GS_W_F16><<<g, 256, 0, s>>>(l.kb[cur], l.tb[cur], l.cb[cur], nnz, n_docs, row_ptr_d,
                                                      fwd_terms_d, fwd_weights_d);
            break;
        default:
            k_unpack_rows<GS_W_U8><<<g, 256, 0, s>>>(l.kb[cur], l.tb[cur], l.cb[cur], nnz, n_docs, row_ptr_d,
                                                     fwd_terms_d, fwd_weights_d);
            break;
    }
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_pack_postings(const int32_t *doc_ids_d, const void *weights_d, int32_t wtype, int64_t n_slots,
                                const int64_t *offsets_d, const int32_t *tile_bounds_d, int32_t vocab, int64_t n_docs,
                                int32_t tile_log2, int32_t w_shift, void *out_d, void *stream) {
    GS_REQUIRE(n_slots >= 0, "n_slots %lld is negative", (long long)n_slots);
    GS_REQUIRE(tile_log2 >= 6 && tile_log2 <= 14, "tile_log2 %d outside [6, 14]", tile_log2);
    GS_REQUIRE(wtype >= GS_W_F32 && wtype <= GS_W_U8, "unknown weight type %d", wtype);
    GS_REQUIRE(wtype == GS_W_U8 || (w_shift >= -200 && w_shift <= 200), "w_shift %d outside [-200, 200]", w_shift);
    GS_REQUIRE(n_slots == 0 || (doc_ids_d && weights_d && out_d), "null pointer");
    GS_REQUIRE(!tile_bounds_d || (offsets_d && vocab > 0 && n_docs >= 0), "tile bounds need offsets, vocab, n_docs");
    if (n_slots == 0) return GS_OK;
    hipStream_t s = gs_stream(stream);
    const unsigned g = gs_blocks(n_slots, 256, 1 << 16);
    uint32_t *out = reinterpret_cast<uint32_t *>(out_d);
    const int64_t n_tiles = (n_docs + (1ll << tile_log2) - 1) >> tile_log2;
    const int64_t pairs = (int64_t)vocab * n_tiles;
    const int64_t arrange_waves = (int64_t)vocab * ((n_tiles + kArrangeTiles - 1) / kArrangeTiles);
    GS_REQUIRE(!tile_bounds_d || arrange_waves <= (int64_t)4 * 0x7FFFFFFF, "too many (term, tile) pairs");
    const unsigned ga = (unsigned)((arrange_waves + 3) / 4);
    // four slots per thread when every array is aligned to that (a weight group of
    // four is 4, 8 or 16 bytes)
    const size_t wbytes = wtype == GS_W_F32 ? 4 : (wtype == GS_W_F16 ? 2 : 1);
    const bool vec = ((uintptr_t)doc_ids_d % 16 == 0) && ((uintptr_t)out_d % 16 == 0) &&
                     ((uintptr_t)weights_d % (4 * wbytes) == 0);
    const unsigned gv = gs_blocks((n_slots + 3) / 4, 256, 1 << 16);
    auto pack = [&](auto wt) {
        constexpr int WT = decltype(wt)::value;
        if (vec) k_pack_postings<WT, true><<<gv, 256, 0, s>>>(doc_ids_d, weights_d, n_slots, tile_log2, w_shift, out);
        else k_pack_postings<WT, false><<<g, 256, 0, s>>>(doc_ids_d, weights_d, n_slots, tile_log2, w_shift, out);
        if (tile_bounds_d && pairs > 0)
            k_pack_arrange<<<ga, 256, 0, s>>>(offsets_d, tile_bounds_d, vocab, n_tiles, out);
    };
    switch (wtype) {
        case GS_W_F32: pack(std::integral_constant<int, GS_W_F32>{}); break;
        case GS_W_F16: pack(std::integral_constant<int, GS_W_F16>{}); break;
        default: w_shift = 0; pack(std::integral_constant<int, GS_W_U8>{}); break;
    }
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_heavy_terms(const int32_t *lengths_d, int32_t vocab, int32_t *heavy_d, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(lengths_d && heavy_d, "null pointer");
    k_heavy_terms<<<1, 1024, 0, gs_stream(stream)>>>(lengths_d, vocab, heavy_d);
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_head_fill(const int32_t *doc_ids_d, const void *weights_d, int32_t wtype, const int64_t *offsets_d,
                            const int32_t *lengths_d, int32_t vocab, const int32_t *heavy_d, int32_t w_shift,
                            int64_t n_docs, int64_t n_rows, int8_t *head_d, int16_t *head_rank_d, void *stream) {
    GS_REQUIRE(vocab > 0, "vocab must be positive, got %d", vocab);
    GS_REQUIRE(n_docs >= 0 && n_rows >= n_docs, "head rows %lld fewer than the %lld docs", (long long)n_rows,
               (long long)n_docs);
    GS_REQUIRE(n_rows % 16 == 0, "head rows %lld not a multiple of 16", (long long)n_rows);
    // gs_search's k_head_scores reads whole GS_HEAD_BLOCK-row blocks up to the
    // last doc's block
    GS_REQUIRE(n_rows >= (n_docs + GS_HEAD_BLOCK - 1) / GS_HEAD_BLOCK * GS_HEAD_BLOCK,
               "head rows %lld fewer than the %lld docs rounded up to GS_HEAD_BLOCK (%d)", (long long)n_rows,
               (long long)n_docs, GS_HEAD_BLOCK);
    GS_REQUIRE(wtype >= GS_W_F32 && wtype <= GS_W_U8, "unknown weight type %d", wtype);
    GS_REQUIRE(wtype == GS_W_U8 || (w_shift >= -200 && w_shift <= 200), "w_shift %d outside [-200, 200]", w_shift);
    GS_REQUIRE(doc_ids_d && weights_d && offsets_d && lengths_d && heavy_d && head_d && head_rank_d,
               "null pointer");
    hipStream_t s = gs_stream(stream);
    k_head_rank<<<gs_blocks(vocab, 256), 256, 0, s>>>(vocab, head_rank_d);
    k_head_rank_set<<<1, kHeavyTerms, 0, s>>>(heavy_d, vocab, head_rank_d);
    GS_CHECK_LAUNCH();
    const int64_t per_wg = (int64_t)kHeadFillBlocks * kHeadFillDocs;
    const int64_t nb = (n_rows + per_wg - 1) / per_wg;  // every row written, zero past n_docs
    if (nb == 0) return GS_OK;
    GS_REQUIRE(nb < (1ll << 31), "too many head rows");
    switch (wtype) {
        case GS_W_F32:
            k_head_fill<GS_W_F32><<<(unsigned)nb, 256, 0, s>>>(doc_ids_d, weights_d, offsets_d, lengths_d, heavy_d,
                                                               w_shift, n_docs, n_rows, head_d);
            break;
        case GS_W_F16:
            k_head_fill<GS_W_F16><<<(unsigned)nb, 256, 0, s>>>(doc_ids_d, weights_d, offsets_d, lengths_d, heavy_d,
                                                               w_shift, n_docs, n_rows, head_d);
            break;
        default:
            k_head_fill<GS_W_U8><<<(unsigned)nb, 256, 0, s>>>(doc_ids_d, weights_d, offsets_d, lengths_d, heavy_d, 0,
                                                              n_docs, n_rows, head_d);
            break;
    }
    GS_CHECK_LAUNCH();
    return GS_OK;
}

extern "C" int gs_pack_shift(float max_abs, int32_t *shift) {
    GS_REQUIRE(shift, "null pointer");
    GS_REQUIRE(std::isfinite(max_abs) && max_abs >= 0.0f, "max_abs %g must be finite and >= 0", (double)max_abs);
    if (max_abs == 0.0f) {
        *shift = 0;
        return GS_OK;
    }
    // max_abs * 2^s is exact in double for every float max_abs and |s| <= 300
    int sh = (int)std::floor(std::log2(8191.0 / (double)max_abs));
    while (std::ldexp((double)max_abs, sh) > 8191.0) --sh;
    while (std::ldexp((double)max_abs, sh + 1) <= 8191.0) ++sh;
    *shift = sh;
    return GS_OK;
}
