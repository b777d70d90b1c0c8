// Dense-row selection (the reference's compacted_topk / torch.topk) and the
// reference's global-atomic scatter-add scoring kernel, on gfx950.
#include "gs_topk.h"

namespace {

using namespace gs;

template <class T>
__global__ void k_fill(T *p, int64_t n, T v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
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
    __shared__ SelStatic sst;
    SelShared sh = sel_view(sst, k);
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

}  // namespace

// ====================================================================== C ABI

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
    GS_CHECK_HIP(sel_attr((const void *)k_select_compacted, sel_lds_bytes(k)));
    k_select_compacted<<<B, kSelThreads, sel_lds_bytes(k), s>>>(scores_d, ld, L, tau_d, cidx, cval, tau_d ? counts_d : nullptr,
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
