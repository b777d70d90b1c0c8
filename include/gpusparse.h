/*
 * gpusparse.h - C ABI of the MI355X (gfx950) exact SPLADE scoring library.
 *
 * The reference (ashutoshuiuc/gpu-sparse) has no native library: its only "FFI"
 * is the Triton JIT launch `kernel[grid](ptrs..., BLOCK_PL=...)`.  Each entry
 * point below replaces one such launch, or a numpy / torch step on the same
 * path, and names the reference code it stands in for.
 *
 * Conventions
 *  - Every pointer argument named *_d is a device pointer (hipMalloc / torch).
 *  - `stream` is a hipStream_t passed as void*; NULL means the null stream.
 *  - No entry point allocates device memory or synchronises the host: scratch
 *    memory is a caller-provided workspace whose size the matching
 *    *_workspace() call reports, and results are produced asynchronously.
 *  - Return value: GS_OK, or an error code with a message from gs_last_error()
 *    (thread-local).  GS_EINVAL maps to ValueError, GS_EHIP to RuntimeError.
 */
#ifndef GPUSPARSE_H
#define GPUSPARSE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_ABI_VERSION 10

#define GS_OK 0
#define GS_EINVAL 1   /* bad argument or layout */
#define GS_EHIP 2     /* HIP runtime error */
#define GS_ENOSPC 3   /* workspace smaller than the *_workspace() size */

/* posting-weight storage types */
#define GS_W_F32 0    /* fp32 weights, fp32 query weights, fp32 tiles, fp64-exact output */
#define GS_W_F16 1    /* IEEE binary16 weights, otherwise as GS_W_F32 */
#define GS_W_U8 2     /* uint8 impacts and uint8 query weights, exact uint32 sums */

/* Per-query status written by gs_search. */
#define GS_ROW_DONE 0
#define GS_ROW_DENSE 1  /* row must be finished by gs_search_dense (rare: overflow or < k positive scores) */

/*
 * Device-resident term-major inverted index: the layout of the reference's
 * GPUInvertedIndex (src/gpu_inverted_index.py:21-35) plus the per-(term, doc
 * tile) posting bounds this library schedules by.
 */
typedef struct gs_index {
    const int32_t *doc_ids_d;     /* [n_slots] doc ids, ascending within each list, -1 padding */
    const void *weights_d;        /* [n_slots] weights in `wtype`, 0 padding */
    const int64_t *offsets_d;     /* [vocab] first slot of each list */
    const int32_t *lengths_d;     /* [vocab] postings per list (before padding) */
    const float *max_abs_d;       /* [vocab] max |weight| per list (0 for empty lists) */
    const int32_t *dup_d;         /* [vocab] equal adjacent doc ids per list (0 when canonical) */
    const int32_t *tile_bounds_d; /* [vocab][n_tiles + 1] list-relative first posting of each doc tile */
    int64_t n_slots;
    int64_t n_docs;
    int32_t vocab;
    int32_t wtype;                /* GS_W_* */
    int32_t tile_log2;            /* docs per tile = 1 << tile_log2 */
    int32_t n_tiles;              /* ceil(n_docs / tile) */
    const int64_t *fwd_ptr_d;     /* optional doc-major copy (gs_forward_fill), used by the exact */
    const int32_t *fwd_terms_d;   /* rescoring of float indexes: [n_docs + 1] row offsets, [nnz] */
    const void *fwd_weights_d;    /* term ids ascending within a row, [nnz] weights; NULL: the
                                     rescoring searches the term lists instead */
    const void *packed_d;         /* optional packed scoring copy (gs_pack_postings) read by the
                                     fused scorer in place of doc_ids_d / weights_d */
    int32_t packed_tile_log2;     /* the tile size packed_d was made for; used only when it equals
                                     tile_log2 */
    int32_t packed_shift;         /* the w_shift packed_d was made with (float weights) */
    const int32_t *heavy_d;       /* optional [GS_HEAVY_TERMS] most frequent terms (gs_heavy_terms):
                                     gs_search then groups queries that share them; NULL: batch order */
    const int8_t *head_d;         /* optional dense copy of the heavy terms' weights (gs_head_fill),
                                     [n_docs rounded up to GS_HEAD_BLOCK][2][GS_HEAVY_TERMS]: with it
                                     (and the packed copy, float weights) gs_search runs the hybrid
                                     search -- heavy terms as int8 matrix products, the rest as LDS adds */
    const int16_t *head_rank_d;   /* [vocab] h for term heavy_d[h], -1 for the others (gs_head_fill) */
} gs_index;

/* Docs per block of the heavy-term products: head_d rows are padded to it. */
#define GS_HEAD_BLOCK 512

/* The heavy terms: the index's GS_HEAVY_TERMS longest lists (gs_heavy_terms).
 * gs_search groups queries by the 64 most frequent of them; the hybrid search
 * takes all of them as int8 matrix products.  64, 128 or 256;
 * gs_heavy_term_count reports the value the library was built with. */
#ifndef GS_HEAVY_TERMS
#define GS_HEAVY_TERMS 64
#endif
int gs_heavy_term_count(void);

/* Tuning knobs of gs_search; zero selects the default. */
typedef struct gs_search_opts {
    int32_t sample_tiles;  /* doc tiles scored first with tau = 0 (all their positive docs become
                              candidates) to seed the k-th-score threshold (default: about 4 k
                              docs, at least 4 Ki and at most 32 Ki docs, widened for batches of
                              few query groups to about 256 workgroups, at most 64 tiles) */
    int32_t cand_cap;      /* candidates kept per query before the dense fallback (0: 2^24 / B within
                              [65536, 2^22], at most the docs rounded up to 256) */
    int32_t unroll;        /* postings per lane per chunk of the fused scorer: 1, 2, 4, 8 or 16 (default
                              16 with a packed copy, else 8) */
    int32_t waves;         /* reserved, ignored */
    void *ev_score_begin;  /* optional hipEvent_t recorded on `stream` right before the fused */
    void *ev_score_end;    /* scoring kernel and right after it (per-kernel timing); may be NULL */
    int32_t tiles_per_wg;  /* consecutive doc tiles walked by one scoring workgroup, 1..64 (default 3
                              when that leaves at least 49152 workgroups, else 2 when that leaves at
                              least 12288, else 1) */
    void **ev_phases;      /* optional array of GS_SEARCH_PHASES hipEvent_t (entries may be NULL)
                              recorded on `stream` at the phase boundaries of gs_search: start,
                              query prep, heavy-term sums (hybrid search; empty otherwise),
                              threshold seed, scoring, candidate selection, fp64 rescoring,
                              final sort; may be NULL */
    int32_t batch_order;   /* 1: score queries in groups of consecutive queries even when the
                              index has heavy_d (default 0: group by shared frequent terms) */
    int32_t no_hybrid;     /* 1: LDS adds for every term even when the index has head_d */
} gs_search_opts;

#define GS_SEARCH_PHASES 8

int gs_query_version(void);
const char *gs_last_error(void);

/* ------------------------------------------------------------ index build
 * Replaces the host numpy builders build_index
 * (lsr_benchmark_engine/gpusparse_retrieval.py:81-115) and
 * build_gpu_index_from_csr (src/run_correctness_verification.py:32-84):
 * stable term-major transpose of a doc-major CSR, lists padded to 32 slots.
 *
 * Step 1, gs_index_count: lengths, padded lengths, exclusive offsets.
 *   info_d[0] <- n_slots (= offsets[V-1] + padded[V-1]),
 *   info_d[1] <- entries whose term id is outside [0, vocab) (build must not proceed).
 * Step 2, gs_index_fill: stable LSD radix sort of (term; doc, weight) by term,
 *   scattered into the padded layout; also max_scores (signed max per list, 0 if
 *   empty: run_correctness_verification.py:63,71) and max_abs.
 */
int gs_index_count(const int32_t *indices_d, int64_t nnz, int32_t vocab, int32_t *lengths_d,
                   int32_t *padded_d, int64_t *offsets_d, int64_t *info_d, void *stream);
size_t gs_index_fill_workspace(int64_t nnz, int32_t vocab);
int gs_index_fill(const int64_t *indptr_d, const int32_t *indices_d, const void *data_d, int32_t wtype,
                  int64_t n_docs, int64_t nnz, int32_t vocab, const int64_t *offsets_d,
                  const int32_t *lengths_d, const int32_t *padded_d, int64_t n_slots,
                  int32_t *doc_ids_d, void *weights_d, float *max_scores_d, float *max_abs_d,
                  void *workspace_d, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------ list checks and bounds
 * gs_check_lists replaces the ascending-doc-id validation of
 * build_chunk_boundaries (src/triton_kernel_chunked.py:96-108) and the invariant
 * check of src/remeasure_2026_09.py:261-299:
 *   bad_d[t] <- 1 if list t has doc[i] < doc[i-1], dup_d[t] <- #(doc[i] == doc[i-1]),
 *   info_d[0] <- number of non-ascending lists, info_d[1] <- number of non-empty lists.
 */
int gs_check_lists(const int32_t *doc_ids_d, const int64_t *offsets_d, const int32_t *lengths_d,
                   int32_t vocab, int32_t *bad_d, int32_t *dup_d, int64_t *info_d, void *stream);

/* Per-list max weight (max_scores of run_correctness_verification.py:63,71: signed
 * max, 0 for empty lists) and max |weight|, for indexes assembled outside
 * gs_index_fill.  Workspace: 8 * vocab bytes. */
int gs_list_max(const void *weights_d, int32_t wtype, const int64_t *offsets_d, const int32_t *lengths_d,
                int32_t vocab, float *max_scores_d, float *max_abs_d, void *workspace_d,
                size_t workspace_bytes, void *stream);

/* Replaces build_chunk_boundaries (src/triton_kernel_chunked.py:110-122):
 *   bounds_d[c][t] = offsets[t] + lower_bound(list t, edge_c), edges = c*doc_chunk
 *   (c < n_chunks) and n_docs; shape [n_chunks + 1][vocab], int64.
 * Lists must be ascending (gs_check_lists). */
int gs_chunk_bounds(const int32_t *doc_ids_d, const int64_t *offsets_d, const int32_t *lengths_d,
                    int32_t vocab, int64_t n_docs, int64_t doc_chunk, int64_t *bounds_d, void *stream);

/* Per-(term, doc tile) bounds used by gs_search: bounds_d[t][j] = lower_bound(list t,
 * j << tile_log2) relative to offsets[t], j = 0..n_tiles; shape [vocab][n_tiles + 1].
 * The reference's per-(term, chunk) sub-ranges at LDS-tile granularity. */
int gs_tile_bounds(const int32_t *doc_ids_d, const int64_t *offsets_d, const int32_t *lengths_d,
                   int32_t vocab, int64_t n_docs, int32_t tile_log2, int32_t *bounds_d, void *stream);

/* Whether every row of a doc-major CSR has non-decreasing column indices (no
 * counterpart in the reference): *unsorted_d = 0 if so, 1 if not.  A CSR whose
 * rows are sorted already is the doc-major copy below (the same rows, term ids
 * ascending, a repeated term's entries in CSR order), so the index build keeps
 * it instead of transposing the index back. */
int gs_rows_sorted(const int64_t *indptr_d, const int32_t *indices_d, int64_t n_rows, int32_t *unsorted_d,
                   void *stream);

/* Doc-major copy of a term-major index, for exact candidate rescoring (the
 * forward-index layout of src/triton_kernel_v4.py:92-158, built on the GPU from
 * the inverted index instead of from a dense matrix).  Row d holds the postings
 * of doc d: row_ptr_d [n_docs + 1] int64 offsets, fwd_terms_d [nnz] int32 term ids
 * ascending within the row (entries of a repeated (doc, term) pair keep their
 * list order), fwd_weights_d [nnz] weights in `wtype`.  nnz = sum of lengths.
 * Doc ids outside [0, n_docs) are left out of every row. */
size_t gs_forward_fill_workspace(int64_t nnz, int32_t vocab);
int gs_forward_fill(const int32_t *doc_ids_d, const void *weights_d, int32_t wtype, const int64_t *offsets_d,
                    const int32_t *lengths_d, int32_t vocab, int64_t n_docs, int64_t nnz, int64_t *row_ptr_d,
                    int32_t *fwd_terms_d, void *fwd_weights_d, void *workspace_d, size_t workspace_bytes,
                    void *stream);

/* Packed scoring copy of the postings (no counterpart in the reference: a layout
 * of its posting arrays for the LDS scorer), one uint32 per slot: the byte offset
 * of its doc's word in a tile slice, (doc mod 2^tile_log2) * 4, in bits 0..15 and
 * the weight in bits 16..31 -- for GS_W_U8 the uint8 weight, for float weights
 * the int16 rint(w * 2^w_shift) (clamped to +-32767; w_shift from gs_pack_shift
 * keeps every |value| <= 8191).  Padding slots (doc id < 0) hold 0.
 * With tile_bounds_d (gs_tile_bounds for this tile_log2; offsets_d, vocab and
 * n_docs of the index) each (term, tile) sub-range is cut into blocks of 1024
 * postings from its start, and the words of each block of more than 64 postings
 * are reordered so that each 64-posting group aligned to the block's start
 * spreads its docs over the 64 residues mod 64 (the LDS banks of their score
 * words): sorted by (doc mod 64, doc), the k-th goes to group k mod G at
 * position k / G while all G groups of the block have room there, then to the
 * first G - 1.  With tile_bounds_d NULL the words stay in slot order.
 * tile_log2 <= 14; w_shift in [-200, 200] (ignored for GS_W_U8). */
int gs_pack_postings(const int32_t *doc_ids_d, const void *weights_d, int32_t wtype, int64_t n_slots,
                     const int64_t *offsets_d, const int32_t *tile_bounds_d, int32_t vocab, int64_t n_docs,
                     int32_t tile_log2, int32_t w_shift, void *out_d, void *stream);
/* The GS_HEAVY_TERMS non-empty posting lists with the most postings (no
 * counterpart in the reference: gs_search's query grouping reads them), as term
 * ids by (length descending, term ascending); -1 past the number of non-empty
 * lists.  lengths_d int32 [vocab] (gs_index.lengths_d), heavy_d int32
 * [GS_HEAVY_TERMS]. */
int gs_heavy_terms(const int32_t *lengths_d, int32_t vocab, int32_t *heavy_d, void *stream);
/* Dense copy of the heavy terms' weights for the hybrid search (no counterpart in
 * the reference: an operand of gs_search's int8 matrix products).  head_d int8
 * [n_rows][2][GS_HEAVY_TERMS], n_rows >= n_docs rounded up to GS_HEAD_BLOCK
 * (gs_search reads that many rows; GS_EINVAL otherwise): row d holds, for h < GS_HEAVY_TERMS, the packed
 * copy's integer weight wq of (d, heavy_d[h]) -- the uint8 weight, or
 * rint(w * 2^w_shift) clamped to +-32767 -- as two limbs, wq & 127 at [d][0][h]
 * and wq >> 7 (arithmetic) at [d][1][h]; 0 where doc d lacks the term.  The
 * heavy lists must hold each doc at most once (gs_check_lists dup = 0) and their
 * |wq| <= 16383 (w_shift from gs_pack_shift keeps every |wq| <= 8191).
 * head_rank_d int16 [vocab] <- h for heavy_d[h], -1 for other terms. */
int gs_head_fill(const int32_t *doc_ids_d, const void *weights_d, int32_t wtype, const int64_t *offsets_d,
                 const int32_t *lengths_d, int32_t vocab, const int32_t *heavy_d, int32_t w_shift,
                 int64_t n_docs, int64_t n_rows, int8_t *head_d, int16_t *head_rank_d, void *stream);
/* Weight scale of a packed copy of float weights: the largest `shift` with
 * max_abs * 2^shift <= 8191, for max_abs = the largest |weight| of the index (0 for
 * max_abs == 0).  GS_EINVAL for a negative or non-finite max_abs. */
int gs_pack_shift(float max_abs, int32_t *shift);

/* ------------------------------------------------------------ search
 * Replaces triton_fused_score (src/triton_kernel.py:159-200) and
 * triton_chunked_score_fused (src/fused_topk.py:106-160): exact top-k of
 *   score[q, d] = sum_j q_weights[q, j] * w(q_terms[q, j], d)
 * over valid terms (0 <= term < vocab; others are skipped as in
 * triton_kernel.py:126-128), ordered by score descending then doc id ascending.
 *   q_terms_d   int32 [B][T] (-1 padding), q_weights_d float32 (or uint8 for GS_W_U8) [B][T]
 *   out_scores_d float32 [B][k] (int32 for GS_W_U8), out_ids_d int64 [B][k]
 *   status_d    int32 [B]: GS_ROW_DONE, or GS_ROW_DENSE when the row has to be
 *               recomputed with gs_search_dense (its outputs are then undefined).
 * Float indexes accumulate fixed-point int32 in LDS doc tiles (from the packed
 * copy: integer products of rint(q * 2^f) and the packed weights) and rescore the
 * selected candidates in fp64 in query-term order, so scores equal the fp64
 * scatter-add rounded to fp32.  1 <= k <= min(n_docs, 8192). */
int gs_search_workspace(const gs_index *index, int32_t B, int32_t T, int32_t k,
                        const gs_search_opts *opts, size_t *bytes);

/* How gs_search would run a batch (no counterpart in the reference: an
 * introspection call for benchmarks and tests). */
typedef struct gs_search_plan_info {
    int32_t seed_tiles;    /* doc tiles scored first with tau = 0 */
    int32_t group_size;    /* queries per scoring group (their slices share one LDS tile) */
    int32_t unroll;        /* postings per lane per chunk */
    int32_t tiles_per_wg;  /* doc tiles per scoring workgroup after the seed tiles */
    int32_t packed;        /* 1 when the scorer reads the packed copy */
    int32_t hybrid;        /* 1 when heavy terms are scored as int8 matrix products (head_d) */
    int32_t cand_cap;      /* candidate slots per query (opts->cand_cap, or the default: 2^24 / B
                              within [65536, 2^22], at most the docs rounded up to 256, at least 2k) */
} gs_search_plan_info;
int gs_search_plan(const gs_index *index, int32_t B, int32_t T, int32_t k, const gs_search_opts *opts,
                   gs_search_plan_info *out);
int gs_search(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B,
              int32_t T, int32_t k, const gs_search_opts *opts, void *out_scores_d,
              int64_t *out_ids_d, int32_t *status_d, void *workspace_d, size_t workspace_bytes,
              void *stream);

/* ------------------------------------------------------------ allocation-free search
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): gs_search with its workspace in a scratch array of the
 * library itself, GS_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load
 * on a GPU until the process ends.  Same arguments (minus the workspace),
 * results and status as gs_search; the caller still passes inputs and outputs.
 * GS_ENOSPC, with a message, when the search needs more scratch than that
 * (gs_search_workspace reports the need): e.g. B = 512, T = 107, k = 1000 fits
 * with cand_cap <= 32768, and B <= 256 fits at the default caps (the hybrid search
 * needs 1.5 bytes more per query slot and doc, for its coarse heavy-term sums).  The scratch
 * keeps the last call's contents; every call clears what it needs cleared.
 * The first call on each device looks up the array's device address
 * (hipGetSymbolAddress): make it outside stream capture.  Later calls record
 * no memset and no allocation or synchronisation, so they can be captured into
 * a HIP graph and replayed (tests/test_zz_no_alloc.py replays one).
 * Calls that overlap on one GPU (other threads, other streams) share that GPU's
 * array and race: serialise them.  Allocates nothing and does not synchronise. */
#define GS_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int gs_search_noalloc(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d, int32_t B,
                      int32_t T, int32_t k, const gs_search_opts *opts, void *out_scores_d, int64_t *out_ids_d,
                      int32_t *status_d, void *stream);

/* Candidate counts of the gs_search that last ran on `workspace_d` with the same
 * (index, B, T, k, opts) (no counterpart in the reference: an introspection call
 * for benchmarks), per scoring slot: cand_d[s] <- docs the fused scorer emitted
 * (before the cand_cap cut), resc_d[s] <- candidates rescored in fp64 (0 for
 * uint8 indexes and for rows flagged GS_ROW_DENSE).  uint32 [B] each; copied on
 * `stream` after the search's kernels. */
int gs_search_counts(const gs_index *index, int32_t B, int32_t T, int32_t k, const gs_search_opts *opts,
                     const void *workspace_d, size_t workspace_bytes, uint32_t *cand_d, uint32_t *resc_d,
                     void *stream);

/* Monolithic exact path (the reference's [B, N] accumulator, triton_kernel.py:182-199):
 * rows listed in rows_d (int32 [R], or NULL for rows 0..B-1) are scored densely
 * over all documents (fp64 or uint32 tiles written to a dense row buffer) and
 * selected exactly; results go to the same rows of out_*.  The workspace bounds
 * how many rows are processed per pass (at least one row must fit).
 * 1 <= k <= n_docs: above 8192 the selection runs in rounds of 8192, each the
 * top of the entries after the previous round's last one. */
int gs_search_dense_workspace(const gs_index *index, int32_t rows_per_pass, size_t *bytes);
int gs_search_dense(const gs_index *index, const int32_t *q_terms_d, const void *q_weights_d,
                    int32_t B, int32_t T, int32_t k, const int32_t *rows_d, int32_t R,
                    void *out_scores_d, int64_t *out_ids_d, void *workspace_d,
                    size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------ dense-row selection
 * Replaces compacted_topk (src/fused_topk.py:71-103) and its
 * _compact_above_threshold_kernel (:33-68): entries of scores_d[B][L] (row stride
 * ld) with value >= tau_d[b] are compacted into a [B][max_cand] candidate buffer,
 * then the top kk = min(k, L) are returned sorted descending (ties: lower column
 * first); missing slots are (-inf, 0).  Rows with more than max_cand candidates
 * are selected from the full row, as the reference's overflow path does.
 * tau_d may be NULL (plain torch.topk semantics on the row).  counts_d int32 [B]
 * receives the per-row candidate count. */
size_t gs_compacted_topk_workspace(int32_t B, int32_t max_cand);
int gs_compacted_topk(const float *scores_d, int64_t ld, int32_t B, int64_t L, const float *tau_d,
                      int32_t k, int32_t max_cand, float *out_values_d, int64_t *out_idx_d,
                      int32_t *counts_d, void *workspace_d, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------ atomic scatter-add
 * The reference's scoring kernel itself: _fast_scatter_add_kernel
 * (src/triton_kernel.py:93-156) when lo_d/hi_d are NULL, and
 * _chunked_scatter_add_kernel (src/triton_kernel_chunked.py:34-80) when they are
 * the [vocab] posting bounds of one chunk.  One program per (query, term) streams
 * the postings and adds q*w into out_d[q*out_stride + doc - chunk_start] with
 * global fp32 atomics (uint32 for GS_W_U8); docs outside [chunk_start,
 * chunk_start + chunk_len) and padding are skipped.  out_d must be pre-zeroed. */
int gs_scatter_add(const gs_index *index, const int64_t *lo_d, const int64_t *hi_d,
                   const int32_t *q_terms_d, const void *q_weights_d, int32_t B, int32_t T,
                   void *out_d, int64_t chunk_start, int64_t chunk_len, int64_t out_stride,
                   int32_t block_pl, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GPUSPARSE_H */
