/*
 * Seeded synthetic SPLADE-like sparse matrices (documents or queries), written
 * straight into CSR arrays.
 *
 * Each row draws from its own counter-seeded SplitMix64 stream, so the output
 * depends only on (seed, stream, row) and never on the thread count.  Per row:
 *   nnz   = clip(rint(exp(mu_n + sigma_n * z)), nnz_min, nnz_max), at most vocab
 *   terms = n_head_forced distinct ranks drawn uniformly from the head_pool most
 *           frequent ranks, then Zipf(s) ranks (p(r) ~ r^-s, r = 1..vocab) drawn
 *           with replacement and rejected when already chosen.  Rejecting repeats
 *           of i.i.d. draws is the same law as successive weighted sampling
 *           without replacement (numpy's choice(replace=False, p=...)).
 *           Term id = rank - 1; ids are written ascending.
 *   w     = min(exp(w_mu + w_sigma * z), w_max) rounded to fp32, one per term in
 *           ascending-id order; stored as fp32, as IEEE binary16 (round to nearest
 *           even), or as uint8 rint(w * 255 / w_max) with zero codes dropped.
 *
 * The generator mirrors the workload description of the reference benchmarks
 * (synthetic Zipf term ids, lognormal weights; cf. the reference's own generator
 * src/gpu_inverted_index.py:137-174), with the distribution parameters of the
 * configurations this project measures.  It is input preparation, not a
 * restatement of any reference algorithm.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    int64_t n_rows;
    int32_t vocab;
    int32_t wmode;        /* 0 = fp32, 1 = fp16 bits, 2 = uint8 code */
    double zipf_s;
    double nnz_mean;      /* mean of the (unclipped) lognormal row length */
    double nnz_sigma;
    int32_t nnz_min, nnz_max;
    double w_mu, w_sigma, w_max;
    int32_t n_head_forced, head_pool;
    uint64_t seed, stream;
} gs_synth_spec;

/* ---------------------------------------------------------------- RNG */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

typedef struct { uint64_t s; } rng_t;

static inline uint64_t rng_next(rng_t *r) {
    r->s += 0x9E3779B97F4A7C15ULL;
    return mix64(r->s);
}

/* uniform double in [0, 1) with 53 random bits */
static inline double rng_u01(rng_t *r) { return (double)(rng_next(r) >> 11) * 0x1.0p-53; }

/* standard normal by Box-Muller (one variate per call; the partner is dropped so
   that every draw consumes exactly two uniforms) */
static inline double rng_normal(rng_t *r) {
    double u1 = 1.0 - rng_u01(r);          /* (0, 1] */
    double u2 = rng_u01(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static inline rng_t row_rng(uint64_t seed, uint64_t stream, int64_t row) {
    rng_t r;
    r.s = mix64(seed ^ mix64(stream + 0x632BE59BD9B4E019ULL) ^ mix64((uint64_t)row * 0xD1B54A32D192ED03ULL + 1));
    return r;
}

/* ---------------------------------------------------------------- fp16 */

/* IEEE binary32 -> binary16 bits, round to nearest even (all ranges). */
uint16_t gs_f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u)                         /* inf / nan */
        return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a >= 0x477FF000u)                         /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (a >= 0x38800000u) {                       /* normal half: >= 2^-14 */
        uint32_t r = a - 0x38000000u;             /* rebias exponent 127 -> 15 */
        uint32_t lsb = (r >> 13) & 1u;
        r += 0x0FFFu + lsb;                       /* round half to even */
        return (uint16_t)(sign | (r >> 13));
    }
    if (a <= 0x33000000u)                         /* <= 2^-25: rounds to +-0 */
        return (uint16_t)sign;
    /* subnormal half: value = m * 2^(e-150), unit 2^-24 */
    uint32_t e = a >> 23;
    uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;                    /* in [14, 24] here */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

/* ---------------------------------------------------------------- Zipf table */

typedef struct {
    int32_t n;
    double *cdf;      /* cdf[r-1] = P(rank <= r) */
    int32_t *guide;   /* guide[i] = first index with cdf >= i / n_guide */
    int32_t n_guide;
} zipf_t;

static int zipf_init(zipf_t *z, int32_t n, double s) {
    z->n = n;
    z->n_guide = n;
    z->cdf = (double *)malloc(sizeof(double) * (size_t)n);
    z->guide = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n + 1));
    if (!z->cdf || !z->guide) return -1;
    double acc = 0.0;
    for (int32_t r = 0; r < n; ++r) {
        acc += pow((double)(r + 1), -s);
        z->cdf[r] = acc;
    }
    for (int32_t r = 0; r < n; ++r) z->cdf[r] /= acc;
    z->cdf[n - 1] = 1.0;
    int32_t j = 0;
    for (int32_t i = 0; i <= n; ++i) {
        double t = (double)i / (double)n;
        while (j < n - 1 && z->cdf[j] < t) ++j;
        z->guide[i] = j;
    }
    return 0;
}

static void zipf_free(zipf_t *z) {
    free(z->cdf);
    free(z->guide);
}

/* index (rank - 1) of one Zipf draw */
static inline int32_t zipf_draw(const zipf_t *z, rng_t *r) {
    double u = rng_u01(r);
    int32_t j = z->guide[(int32_t)(u * (double)z->n_guide)];
    while (z->cdf[j] <= u && j < z->n - 1) ++j;
    return j;
}

/* ---------------------------------------------------------------- rows */

static int cmp_i32(const void *a, const void *b) {
    int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return (x > y) - (x < y);
}

/* Generates one row into terms[] / codes[] (codes: fp32 bits, fp16 bits or u8).
   Returns the number of stored entries (uint8 rows drop zero codes). */
static int32_t gen_row(const gs_synth_spec *sp, const zipf_t *z, int64_t row, uint8_t *bitmap,
                       int32_t *terms, uint32_t *codes) {
    rng_t r = row_rng(sp->seed, sp->stream, row);
    const int32_t V = sp->vocab;
    double sig = sp->nnz_sigma;
    double mu = log(sp->nnz_mean) - 0.5 * sig * sig;
    double len = rint(exp(mu + sig * rng_normal(&r)));
    if (len < sp->nnz_min) len = sp->nnz_min;
    if (len > sp->nnz_max) len = sp->nnz_max;
    int32_t n = (int32_t)len;
    if (n > V) n = V;

    int32_t cnt = 0;
    int32_t pool = sp->head_pool < V ? sp->head_pool : V;
    int32_t forced = sp->n_head_forced < n ? sp->n_head_forced : n;
    if (forced > pool) forced = pool;
    while (cnt < forced) {
        int32_t t = (int32_t)(rng_u01(&r) * (double)pool);
        if (!(bitmap[t >> 3] & (1u << (t & 7)))) {
            bitmap[t >> 3] |= (uint8_t)(1u << (t & 7));
            terms[cnt++] = t;
        }
    }
    while (cnt < n) {
        int32_t t = zipf_draw(z, &r);
        if (!(bitmap[t >> 3] & (1u << (t & 7)))) {
            bitmap[t >> 3] |= (uint8_t)(1u << (t & 7));
            terms[cnt++] = t;
        }
    }
    for (int32_t i = 0; i < cnt; ++i) bitmap[terms[i] >> 3] = 0;
    qsort(terms, (size_t)cnt, sizeof(int32_t), cmp_i32);

    int32_t out = 0;
    for (int32_t i = 0; i < cnt; ++i) {
        double w = exp(sp->w_mu + sp->w_sigma * rng_normal(&r));
        if (w > sp->w_max) w = sp->w_max;
        float wf = (float)w;
        uint32_t code;
        if (sp->wmode == 0) {
            memcpy(&code, &wf, 4);
        } else if (sp->wmode == 1) {
            code = gs_f32_to_f16_bits(wf);
        } else {
            double qv = rint((double)wf * 255.0 / sp->w_max);
            if (qv <= 0.0) continue;            /* zero impact: dropped */
            code = (uint32_t)(qv > 255.0 ? 255.0 : qv);
        }
        terms[out] = terms[i];
        codes[out] = code;
        ++out;
    }
    return out;
}

static int check_spec(const gs_synth_spec *sp) {
    if (sp->n_rows < 0 || sp->vocab <= 0 || sp->nnz_min < 0 || sp->nnz_max < sp->nnz_min ||
        sp->wmode < 0 || sp->wmode > 2 || sp->nnz_mean <= 0.0 || sp->w_max <= 0.0)
        return -1;
    return 0;
}

/* Pass 1: stored entries per row.  Returns the total, or -1 on a bad spec. */
int64_t gs_synth_count(const gs_synth_spec *sp, int64_t *row_nnz, int nthreads) {
    if (check_spec(sp)) return -1;
    zipf_t z;
    if (zipf_init(&z, sp->vocab, sp->zipf_s)) return -1;
    int64_t total = 0;
    int bad = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) reduction(+ : total)
    {
        int cap = sp->nnz_max < sp->vocab ? sp->nnz_max : sp->vocab;
        uint8_t *bm = (uint8_t *)calloc((size_t)(sp->vocab / 8 + 1), 1);
        int32_t *terms = (int32_t *)malloc(sizeof(int32_t) * (size_t)(cap + 1));
        uint32_t *codes = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(cap + 1));
        if (!bm || !terms || !codes) {
#pragma omp atomic write
            bad = 1;
        } else {
#pragma omp for schedule(dynamic, 4096)
            for (int64_t row = 0; row < sp->n_rows; ++row) {
                int32_t n = gen_row(sp, &z, row, bm, terms, codes);
                row_nnz[row] = n;
                total += n;
            }
        }
        free(bm);
        free(terms);
        free(codes);
    }
    zipf_free(&z);
    return bad ? -1 : total;
}

/* Pass 2: fills indices / data for rows given indptr (exclusive scan of pass 1).
   data is float*, uint16_t* or uint8_t* according to wmode. */
int gs_synth_fill(const gs_synth_spec *sp, const int64_t *indptr, int32_t *indices, void *data,
                  int nthreads) {
    if (check_spec(sp)) return -1;
    zipf_t z;
    if (zipf_init(&z, sp->vocab, sp->zipf_s)) return -1;
    int bad = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        int cap = sp->nnz_max < sp->vocab ? sp->nnz_max : sp->vocab;
        uint8_t *bm = (uint8_t *)calloc((size_t)(sp->vocab / 8 + 1), 1);
        int32_t *terms = (int32_t *)malloc(sizeof(int32_t) * (size_t)(cap + 1));
        uint32_t *codes = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(cap + 1));
        if (!bm || !terms || !codes) {
#pragma omp atomic write
            bad = 1;
        } else {
#pragma omp for schedule(dynamic, 4096)
            for (int64_t row = 0; row < sp->n_rows; ++row) {
                int32_t n = gen_row(sp, &z, row, bm, terms, codes);
                int64_t o = indptr[row];
                if (indptr[row + 1] - o != n) {
#pragma omp atomic write
                    bad = 1;
                    continue;
                }
                memcpy(indices + o, terms, sizeof(int32_t) * (size_t)n);
                if (sp->wmode == 0) {
                    memcpy((uint32_t *)data + o, codes, sizeof(uint32_t) * (size_t)n);
                } else if (sp->wmode == 1) {
                    uint16_t *d = (uint16_t *)data + o;
                    for (int32_t i = 0; i < n; ++i) d[i] = (uint16_t)codes[i];
                } else {
                    uint8_t *d = (uint8_t *)data + o;
                    for (int32_t i = 0; i < n; ++i) d[i] = (uint8_t)codes[i];
                }
            }
        }
        free(bm);
        free(terms);
        free(codes);
    }
    zipf_free(&z);
    return bad ? -1 : 0;
}

/* Converts n fp32 values to binary16 bits (round to nearest even). */
void gs_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n, int nthreads) {
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
    for (int64_t i = 0; i < n; ++i) dst[i] = gs_f32_to_f16_bits(src[i]);
}
