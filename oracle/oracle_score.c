/*
 * CPU oracle scorer.  TEST INFRASTRUCTURE ONLY: loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product path.
 *
 * orc_search restates the exact scatter-add of the reference kernel
 * (src/triton_kernel.py:142-156: out[q, doc] += wq * w over every posting of
 * every valid query term, terms < 0 or >= vocab skipped as at :126-128),
 * accumulated in float64 (uint64 for uint8 impacts) in query-term then posting
 * order, followed by an exact top-k ordered by score descending, doc id
 * ascending (a heap over all num_docs documents, so zero-score documents fill the
 * list as in torch.topk over the dense row at :199).
 *
 * orc_cpu_sequential restates the reference CPU path cpu_sequential_score
 * (src/gpu_scoring.py:221-259): one float32 accumulator per query,
 * doc_scores[doc] += q * w (the product rounded to float32), then top-k.  It
 * is the timed CPU baseline.  uint8 impacts accumulate in uint32.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int shift = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                ++shift;
            }
            m &= 0x3FFu;
            bits = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline double weight_at(const void *w, int wtype, int64_t i) {
    if (wtype == 0) return (double)((const float *)w)[i];
    if (wtype == 1) return (double)half_to_float(((const uint16_t *)w)[i]);
    return (double)((const uint8_t *)w)[i];
}

typedef struct {
    double s;
    int64_t d;
} entry_t;

/* a is ranked before b: larger score, then smaller doc id */
static inline int before(entry_t a, entry_t b) { return a.s > b.s || (a.s == b.s && a.d < b.d); }

/* min-heap on rank: root = the entry ranked last */
static void heap_down(entry_t *h, int n, int i) {
    for (;;) {
        int l = 2 * i + 1, r = l + 1, w = i;
        if (l < n && before(h[w], h[l])) w = l;
        if (r < n && before(h[w], h[r])) w = r;
        if (w == i) return;
        entry_t t = h[i];
        h[i] = h[w];
        h[w] = t;
        i = w;
    }
}

static int cmp_entry(const void *a, const void *b) {
    entry_t x = *(const entry_t *)a, y = *(const entry_t *)b;
    if (before(x, y)) return -1;
    if (before(y, x)) return 1;
    return 0;
}

/* top-k of scores[0..n) (as doubles) by (score desc, doc asc) */
static void topk_double(const double *scores, int64_t n, int k, entry_t *heap, double *out_s, int64_t *out_i) {
    int m = 0;
    for (int64_t d = 0; d < n; ++d) {
        entry_t e = {scores[d], d};
        if (m < k) {
            heap[m++] = e;
            if (m == k)
                for (int i = k / 2 - 1; i >= 0; --i) heap_down(heap, k, i);
        } else if (before(e, heap[0])) {
            heap[0] = e;
            heap_down(heap, k, 0);
        }
    }
    qsort(heap, (size_t)m, sizeof(entry_t), cmp_entry);
    for (int i = 0; i < m; ++i) {
        out_s[i] = heap[i].s;
        out_i[i] = heap[i].d;
    }
}

int orc_search(const int32_t *doc, const void *w, int wtype, const int64_t *off, const int32_t *len, int32_t V,
               int64_t N, const int32_t *qt, const void *qw, int32_t B, int32_t T, int32_t k, double *out_s,
               int64_t *out_i, void *unused, int threads) {
    (void)unused;
    if (k < 1 || k > N || B < 0 || T < 0) return 1;
    int bad = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        double *acc = (double *)malloc(sizeof(double) * (size_t)N);
        uint64_t *iacc = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)N);
        entry_t *heap = (entry_t *)malloc(sizeof(entry_t) * (size_t)k);
        if (!acc || !iacc || !heap) {
#pragma omp atomic write
            bad = 2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int32_t q = 0; q < B; ++q) {
                if (wtype == 2) {
                    memset(iacc, 0, sizeof(uint64_t) * (size_t)N);
                    for (int32_t j = 0; j < T; ++j) {
                        int32_t t = qt[(int64_t)q * T + j];
                        if (t < 0 || t >= V) continue;
                        uint64_t wq = ((const uint8_t *)qw)[(int64_t)q * T + j];
                        const int32_t *dp = doc + off[t];
                        const uint8_t *wp = (const uint8_t *)w + off[t];
                        for (int32_t p = 0; p < len[t]; ++p) iacc[dp[p]] += wq * (uint64_t)wp[p];
                    }
                    for (int64_t d = 0; d < N; ++d) acc[d] = (double)iacc[d];
                } else {
                    memset(acc, 0, sizeof(double) * (size_t)N);
                    for (int32_t j = 0; j < T; ++j) {
                        int32_t t = qt[(int64_t)q * T + j];
                        if (t < 0 || t >= V) continue;
                        double wq = (double)((const float *)qw)[(int64_t)q * T + j];
                        const int32_t *dp = doc + off[t];
                        for (int32_t p = 0; p < len[t]; ++p) acc[dp[p]] += wq * weight_at(w, wtype, off[t] + p);
                    }
                }
                topk_double(acc, N, k, heap, out_s + (int64_t)q * k, out_i + (int64_t)q * k);
            }
        }
        free(acc);
        free(iacc);
        free(heap);
    }
    return bad;
}

int orc_cpu_sequential(const int32_t *doc, const void *w, int wtype, const int64_t *off, const int32_t *len,
                       int32_t V, int64_t N, const int32_t *qt, const void *qw, int32_t B, int32_t T, int32_t k,
                       float *out_s, int64_t *out_i, int threads) {
    if (k < 1 || k > N || B < 0 || T < 0) return 1;
    int bad = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)N);
        uint32_t *iacc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)N);
        double *tmp = (double *)malloc(sizeof(double) * (size_t)k);
        entry_t *heap = (entry_t *)malloc(sizeof(entry_t) * (size_t)k);
        if (!acc || !iacc || !tmp || !heap) {
#pragma omp atomic write
            bad = 2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int32_t q = 0; q < B; ++q) {
                int m = 0;
                if (wtype == 2) {
                    memset(iacc, 0, sizeof(uint32_t) * (size_t)N);
                    for (int32_t j = 0; j < T; ++j) {
                        int32_t t = qt[(int64_t)q * T + j];
                        if (t < 0 || t >= V) continue;
                        uint32_t wq = ((const uint8_t *)qw)[(int64_t)q * T + j];
                        const int32_t *dp = doc + off[t];
                        const uint8_t *wp = (const uint8_t *)w + off[t];
                        for (int32_t p = 0; p < len[t]; ++p) iacc[dp[p]] += wq * (uint32_t)wp[p];
                    }
                    for (int64_t d = 0; d < N; ++d) {
                        entry_t e = {(double)iacc[d], d};
                        if (m < k) {
                            heap[m++] = e;
                            if (m == k)
                                for (int i = k / 2 - 1; i >= 0; --i) heap_down(heap, k, i);
                        } else if (before(e, heap[0])) {
                            heap[0] = e;
                            heap_down(heap, k, 0);
                        }
                    }
                } else {
                    memset(acc, 0, sizeof(float) * (size_t)N);
                    for (int32_t j = 0; j < T; ++j) {
                        int32_t t = qt[(int64_t)q * T + j];
                        if (t < 0 || t >= V) continue;
                        float wq = ((const float *)qw)[(int64_t)q * T + j];
                        const int32_t *dp = doc + off[t];
                        if (wtype == 0) {
                            const float *wp = (const float *)w + off[t];
                            for (int32_t p = 0; p < len[t]; ++p) acc[dp[p]] += wq * wp[p];
                        } else {
                            const uint16_t *wp = (const uint16_t *)w + off[t];
                            for (int32_t p = 0; p < len[t]; ++p) acc[dp[p]] += wq * half_to_float(wp[p]);
                        }
                    }
                    for (int64_t d = 0; d < N; ++d) {
                        entry_t e = {(double)acc[d], d};
                        if (m < k) {
                            heap[m++] = e;
                            if (m == k)
                                for (int i = k / 2 - 1; i >= 0; --i) heap_down(heap, k, i);
                        } else if (before(e, heap[0])) {
                            heap[0] = e;
                            heap_down(heap, k, 0);
                        }
                    }
                }
                qsort(heap, (size_t)m, sizeof(entry_t), cmp_entry);
                for (int i = 0; i < m; ++i) {
                    out_s[(int64_t)q * k + i] = (float)heap[i].s;
                    out_i[(int64_t)q * k + i] = heap[i].d;
                }
            }
        }
        free(acc);
        free(iacc);
        free(tmp);
        free(heap);
    }
    return bad;
}

/*
 * Order-independent checksum of a posting multiset: the sum (mod 2^64) over
 * postings of mix(doc, term, weight bits), with mix a SplitMix64-style finaliser.
 * Two collections of (doc, term, weight) triples agree on it when they hold the
 * same triples; any lost, duplicated, moved or altered posting changes it with
 * probability 1 - 2^-64.  Used to check a full-size GPU index against the CSR it
 * was built from without a host rebuild.
 */
static uint64_t mix3(uint64_t d, uint64_t t, uint64_t w) {
    uint64_t h = d * 0x9E3779B97F4A7C15ull ^ (t + 0x632BE59BD9B4E019ull) * 0xC2B2AE3D27D4EB4Full ^
                 (w + 0x8CB92BA72F3D8DD7ull) * 0x165667B19E3779F9ull;
    h ^= h >> 31;
    h *= 0xBF58476D1CE4E5B9ull;
    h ^= h >> 29;
    h *= 0x94D049BB133111EBull;
    return h ^ (h >> 32);
}

static uint64_t wbits(const void *w, int wtype, int64_t i) {
    if (wtype == 0) return ((const uint32_t *)w)[i];
    if (wtype == 1) return ((const uint16_t *)w)[i];
    return ((const uint8_t *)w)[i];
}

/* CSR rows = docs, columns = terms. */
uint64_t orc_checksum_csr(const int64_t *indptr, const int32_t *indices, const void *data, int wtype, int64_t n_rows,
                          int threads) {
    uint64_t sum = 0;
#pragma omp parallel for schedule(dynamic, 4096) reduction(+ : sum) num_threads(threads > 0 ? threads : 1)
    for (int64_t d = 0; d < n_rows; ++d)
        for (int64_t i = indptr[d]; i < indptr[d + 1]; ++i)
            sum += mix3((uint64_t)d, (uint64_t)(uint32_t)indices[i], wbits(data, wtype, i));
    return sum;
}

/* Term-major index: list t = slots [off[t], off[t] + len[t]).  *bad_pad <- number
 * of slots in [off[t] + len[t], off[t] + padded[t]) that are not (-1, 0), plus
 * list slots holding a negative doc id. */
uint64_t orc_checksum_index(const int32_t *doc, const void *w, int wtype, const int64_t *off, const int32_t *len,
                            const int32_t *padded, int32_t V, int threads, int64_t *bad_pad) {
    uint64_t sum = 0;
    int64_t bad = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : sum, bad) num_threads(threads > 0 ? threads : 1)
    for (int32_t t = 0; t < V; ++t) {
        for (int64_t i = off[t]; i < off[t] + len[t]; ++i) {
            if (doc[i] < 0) ++bad;
            sum += mix3((uint64_t)(uint32_t)doc[i], (uint64_t)t, wbits(w, wtype, i));
        }
        for (int64_t i = off[t] + len[t]; i < off[t] + padded[t]; ++i)
            if (doc[i] != -1 || wbits(w, wtype, i) != 0) ++bad;
    }
    *bad_pad = bad;
    return sum;
}
