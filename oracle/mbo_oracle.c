/*
 * mbo_oracle.c — CPU restatement of MacBoost's tree-build hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the reference results the HIP path in
 * macboost_amd/ is compared with, and the timed CPU baseline of bench.py.
 * The shipped library never links or calls it.
 *
 * Plain C11 with OpenMP, IEEE float semantics (built with
 * -ffp-contract=off, no fast-math).  Threads split only work whose result
 * does not depend on the split: per-feature or per-row independent loops,
 * integer histogram sums and maxima of f32 bit patterns, so the results
 * are bit-identical at any thread count (orc_set_threads(1) is the scalar
 * baseline).  Each function names the reference file:line it follows.  Two deliberate, documented restatements:
 *   1. Histogram sums are exact int64 totals of the quantised gradient words
 *      and every split candidate is dequantised once from the exact integer
 *      prefix (reference: per-4096-row-group float dequantisation + float
 *      atomics + float prefix sums, Shaders.swift:257-285, :427-428).
 *   2. exp() in the logistic/poisson/tweedie gradients is evaluated in double
 *      and rounded to float once (reference: Metal fast-math expf,
 *      Shaders.swift:110, :122, :127), so the GPU and this oracle agree to the
 *      bit except on double-rounding ties.
 * Node counts (cover, liveness, which sibling is built) come from the row
 * partition; the reference reads the same integers from a count channel of
 * the histogram (Shaders.swift:1406-1423).
 */
#include "mbo_oracle.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

void orc_set_threads(int32_t n) { omp_set_num_threads(n > 0 ? n : omp_get_num_procs()); }
int32_t orc_get_threads(void) { return omp_get_max_threads(); }

#define PI_F 3.14159274101257324f   /* Float.pi */
#define GOLDEN 0x9E3779B97F4A7C15ULL

/* ------------------------------------------------------------------------ */
/* SplitMix64 and generators: DataGen.swift:6-26, :68-94                     */
/* ------------------------------------------------------------------------ */

uint64_t orc_splitmix_next(uint64_t *s) {          /* DataGen.swift:10-16 */
    *s += GOLDEN;
    uint64_t z = *s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float orc_splitmix_uniform(uint64_t *s) {         /* DataGen.swift:18-20 */
    return (float)(orc_splitmix_next(s) >> 40) * (1.0f / 16777216.0f);
}

float orc_splitmix_normal(uint64_t *s) {          /* DataGen.swift:22-25 */
    float u1 = orc_splitmix_uniform(s);
    if (u1 < 1e-7f) u1 = 1e-7f;
    float u2 = orc_splitmix_uniform(s);
    return sqrtf(-2.0f * logf(u1)) * cosf(2.0f * PI_F * u2);
}

void orc_friedman(int64_t rows, int32_t cols, uint64_t seed, float noise,
                  float *x, float *y) {           /* DataGen.swift:68-94 */
    if (cols < 5 || rows <= 0) return;              /* precondition(cols >= 5) */
    for (int32_t f = 0; f < cols; ++f) {
        uint64_t s = seed + (uint64_t)f * GOLDEN;
        float *col = x + (int64_t)f * rows;
        for (int64_t i = 0; i < rows; ++i) col[i] = orc_splitmix_uniform(&s);
    }
    const int64_t chunk = 65536;
    int64_t nchunks = (rows + chunk - 1) / chunk;
    for (int64_t c = 0; c < nchunks; ++c) {
        uint64_t s = (seed ^ 0xDEADBEEFULL) + (uint64_t)c * GOLDEN;
        int64_t end = (c + 1) * chunk < rows ? (c + 1) * chunk : rows;
        for (int64_t i = c * chunk; i < end; ++i) {
            float x0 = x[i], x1 = x[rows + i], x2 = x[2 * rows + i];
            float x3 = x[3 * rows + i], x4 = x[4 * rows + i];
            float v = 10.0f * sinf(PI_F * x0 * x1);
            v = v + 20.0f * (x2 - 0.5f) * (x2 - 0.5f);
            v = v + 10.0f * x3;
            v = v + 5.0f * x4;
            y[i] = v + noise * orc_splitmix_normal(&s);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Binning: Binner.swift:33-56 (edges), Shaders.swift:46-76 (bin_data)       */
/* ------------------------------------------------------------------------ */

static int cmp_float(const void *a, const void *b) {
    float x = *(const float *)a, y = *(const float *)b;
    return (x > y) - (x < y);
}

void orc_compute_edges_planted(const float *x, int64_t rows, int32_t cols, int64_t rs,
                               int64_t cs, int32_t num_bins, const uint8_t *is_cat,
                               int64_t sample_cap, float *edges, int32_t plant) {
    /* Binner.swift:27-30: dataBins = numBins - 1 (the last bin is the missing
     * bin), numEdges = dataBins - 1, step = max(1, rows / sampleCap). */
    int32_t data_bins = num_bins - 1, num_edges = data_bins - 1;
    int64_t step = rows / sample_cap;
    if (plant == ORC_PLANT_EDGE_CEIL) step = (rows + sample_cap - 1) / sample_cap;
    if (plant == ORC_PLANT_EDGE_NOSTRIDE) step = 1;
    if (step < 1) step = 1;
    memset(edges, 0, sizeof(float) * (size_t)cols * (size_t)num_edges);
#pragma omp parallel
    {
        float *sample = (float *)malloc(sizeof(float) * (size_t)(rows / step + 1));
#pragma omp for schedule(dynamic, 1)
        for (int32_t f = 0; f < cols; ++f) {
            if (is_cat && is_cat[f]) continue;        /* Binner.swift:36 */
            /* Binner.swift:37-44: rows 0, step, 2*step, ... ; NaN skipped */
            int64_t m = 0;
            for (int64_t i = 0; i < rows; i += step) {
                float v = x[i * rs + (int64_t)f * cs];
                if (!isnan(v)) sample[m++] = v;
            }
            if (m == 0) continue;                     /* all-NaN column: edges stay 0 */
            qsort(sample, (size_t)m, sizeof(float), cmp_float);
            /* Binner.swift:48-51: edge k = sample[min(m-1, (k+1)*m / dataBins)];
             * k + 1 <= dataBins - 1, so the index never passes m - 1 */
            for (int32_t k = 0; k < num_edges; ++k) {
                int64_t num = (int64_t)(k + 1) * m, den = data_bins;
                if (plant == ORC_PLANT_EDGE_K) num = (int64_t)k * m;
                if (plant == ORC_PLANT_EDGE_K2) num = (int64_t)(k + 2) * m;
                if (plant == ORC_PLANT_EDGE_NUMBINS) den = num_bins;
                if (plant == ORC_PLANT_EDGE_M1) num = (int64_t)(k + 1) * (m - 1);
                int64_t idx = num / den;
                if (idx > m - 1) idx = m - 1;
                edges[(int64_t)f * num_edges + k] = sample[idx];
            }
        }
        free(sample);
    }
}

void orc_compute_edges(const float *x, int64_t rows, int32_t cols, int64_t rs,
                       int64_t cs, int32_t num_bins, const uint8_t *is_cat,
                       int64_t sample_cap, float *edges) {
    orc_compute_edges_planted(x, rows, cols, rs, cs, num_bins, is_cat, sample_cap, edges, 0);
}

uint8_t orc_bin_value(float v, const float *e, int32_t num_bins, int is_cat) {
    int32_t data_bins = num_bins - 1;
    if (isnan(v)) return (uint8_t)data_bins;
    if (is_cat) {
        int c = (int)rintf(v);
        if (c < 0) c = 0;
        if (c > data_bins - 1) c = data_bins - 1;
        return (uint8_t)c;
    }
    uint32_t lo = 0, hi = (uint32_t)(data_bins - 1);
    while (lo < hi) {
        uint32_t mid = (lo + hi) >> 1;
        if (v > e[mid]) lo = mid + 1; else hi = mid;
    }
    return (uint8_t)lo;
}

void orc_bin_matrix(const float *x, int64_t rows, int32_t cols, int64_t rs, int64_t cs,
                    const float *edges, const uint8_t *is_cat, int32_t num_bins,
                    uint8_t *bins_fm) {
    int32_t num_edges = num_bins - 2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int32_t f = 0; f < cols; ++f) {
        const float *e = edges + (int64_t)f * num_edges;
        int c = is_cat ? is_cat[f] : 0;
        for (int64_t i = 0; i < rows; ++i)
            bins_fm[(int64_t)f * rows + i] =
                orc_bin_value(x[i * rs + (int64_t)f * cs], e, num_bins, c);
    }
}

/* ------------------------------------------------------------------------ */
/* Base score: Booster.swift:775-848.  Means are accumulated in double and   */
/* rounded once (the reference uses vDSP, whose order is unspecified).      */
/* ------------------------------------------------------------------------ */

/* Sums over every row are taken in blocks of 65,536 rows, each block in a
 * fixed order: 64 partial sums in double, partial l adding rows l, l + 64,
 * l + 128, ... of the block in row order, then partial l adds partial l + s
 * for s = 32, 16, 8, 4, 2, 1 (partial 0 is the block's sum); then the block
 * sums in block order (the reference's vDSP sums leave the order
 * unspecified; the library's device reduction uses this one). */
#define ORC_SUM_BLOCK 65536

static void orc_block_sums(const float *y, const float *w, int64_t rows, int32_t obj, double spw,
                           int64_t b, double *out1, double *out2) {
    double a1[64], a2[64];
    for (int l = 0; l < 64; ++l) { a1[l] = 0.0; a2[l] = 0.0; }
    const int64_t lo = b * ORC_SUM_BLOCK;
    const int64_t hi = lo + ORC_SUM_BLOCK < rows ? lo + ORC_SUM_BLOCK : rows;
    for (int64_t r = lo; r < hi; r += 64) {
        for (int l = 0; l < 64 && r + l < hi; ++l) {
            const int64_t i = r + l;
            const double wi = w ? (double)w[i] : 1.0;
            if (obj == ORC_OBJ_LOGISTIC) {
                if (y[i] > 0.5f) { a1[l] += wi * spw; a2[l] += wi * spw; } else a2[l] += wi;
            } else {
                a1[l] += wi * (double)y[i];
                a2[l] += wi;
            }
        }
    }
    for (int s = 32; s >= 1; s >>= 1)
        for (int l = 0; l < s; ++l) { a1[l] += a1[l + s]; a2[l] += a2[l + s]; }
    *out1 = a1[0];
    *out2 = a2[0];
}

float orc_base_score(const float *y, const float *w, int64_t rows, int32_t obj, float spw) {
    const int64_t nblk = (rows + ORC_SUM_BLOCK - 1) / ORC_SUM_BLOCK;
    double *s1 = (double *)calloc((size_t)(nblk > 0 ? nblk : 1), sizeof(double));
    double *s2 = (double *)calloc((size_t)(nblk > 0 ? nblk : 1), sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t b = 0; b < nblk; ++b) orc_block_sums(y, w, rows, obj, (double)spw, b, &s1[b], &s2[b]);
    double a = 0, c = 0;
    for (int64_t b = 0; b < nblk; ++b) { a += s1[b]; c += s2[b]; }
    free(s1); free(s2);
    if (obj == ORC_OBJ_LOGISTIC) {
        float p = (float)(a / (c > 1e-12 ? c : 1e-12));
        if (p < 1e-6f) p = 1e-6f;
        if (p > 1.0f - 1e-6f) p = 1.0f - 1e-6f;
        return logf(p / (1.0f - p));
    }
    float m = c > 0 ? (float)(a / c) : 0.0f;
    if (obj == ORC_OBJ_POISSON || obj == ORC_OBJ_TWEEDIE) return logf(m);
    return m;
}

/* subsampleQuantile (Booster.swift:786-794): the base score of the L1 and
 * quantile objectives, from every max(1, rows/200000)-th label. */
float orc_label_quantile(const float *y, int64_t rows, float q) {
    int64_t step = rows / 200000;
    if (step < 1) step = 1;
    float *s = (float *)malloc(sizeof(float) * (size_t)(rows / step + 1));
    int64_t m = 0;
    for (int64_t i = 0; i < rows; i += step) s[m++] = y[i];
    qsort(s, (size_t)m, sizeof(float), cmp_float);
    int64_t idx = (int64_t)((float)m * q);
    if (idx > m - 1) idx = m - 1;
    float v = s[idx];
    free(s);
    return v;
}

/* ------------------------------------------------------------------------ */
/* Gradients + maxima (Shaders.swift:87-138), quantisation (:176-192)       */
/* ------------------------------------------------------------------------ */

static inline float exp_via_double(float x) { return (float)exp((double)x); }
static inline float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }
static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

void orc_gradients(const float *preds, const float *y, const float *w, int64_t rows,
                   int32_t obj, float alpha, float aux, float *g_out, float *h_out,
                   float *max_g, float *max_h) {
    uint32_t mg = 0, mh = 0;   /* max taken on the f32 bit patterns, :87-94 */
#pragma omp parallel for schedule(static) reduction(max : mg, mh)
    for (int64_t i = 0; i < rows; ++i) {
        float f = preds[i], yy = y[i], g, h;
        switch (obj) {
        case ORC_OBJ_LOGISTIC: {
            float q = 1.0f / (1.0f + exp_via_double(-f));
            float ww = yy > 0.5f ? aux : 1.0f;
            g = (q - yy) * ww;
            h = fmaxf(q * (1.0f - q), 1e-6f) * ww;
            break;
        }
        case ORC_OBJ_MAE: g = f > yy ? 1.0f : -1.0f; h = 1.0f; break;
        case ORC_OBJ_HUBER: g = clampf(f - yy, -alpha, alpha); h = 1.0f; break;
        case ORC_OBJ_QUANTILE: g = f > yy ? (1.0f - alpha) : -alpha; h = 1.0f; break;
        case ORC_OBJ_POISSON: {
            float mu = exp_via_double(clampf(f, -30.0f, 30.0f));
            g = mu - yy; h = fmaxf(mu, 1e-6f);
            break;
        }
        case ORC_OBJ_TWEEDIE: {
            float fc = clampf(f, -30.0f, 30.0f);
            float e2 = exp_via_double((2.0f - aux) * fc), e1 = exp_via_double((1.0f - aux) * fc);
            g = e2 - yy * e1;
            h = fmaxf((2.0f - aux) * e2 - (1.0f - aux) * yy * e1, 1e-6f);
            break;
        }
        default: g = f - yy; h = 1.0f; break;
        }
        if (w) { g *= w[i]; h *= w[i]; }
        g_out[i] = g; h_out[i] = h;
        uint32_t ag = fbits(fabsf(g)), hh = fbits(h);
        if (ag > mg) mg = ag;
        if (hh > mh) mh = hh;
    }
    *max_g = bitsf(mg);
    *max_h = bitsf(mh);
}

void orc_gradients_mc(const float *preds, const float *y, const float *w, int64_t rows,
                      int32_t K, int32_t cls, float *g_out, float *h_out, float *max_g,
                      float *max_h) {
    uint32_t mg = 0, mh = 0;
    for (int64_t i = 0; i < rows; ++i) {
        float m = -INFINITY;
        for (int32_t k = 0; k < K; ++k) m = fmaxf(m, preds[(int64_t)k * rows + i]);
        float sum = 0.0f;
        for (int32_t k = 0; k < K; ++k) sum += exp_via_double(preds[(int64_t)k * rows + i] - m);
        float pk = exp_via_double(preds[(int64_t)cls * rows + i] - m) / sum;
        float yk = (int32_t)y[i] == cls ? 1.0f : 0.0f;
        float g = pk - yk;
        float h = fmaxf(2.0f * pk * (1.0f - pk), 1e-6f);
        if (w) { g *= w[i]; h *= w[i]; }
        g_out[i] = g; h_out[i] = h;
        uint32_t ag = fbits(fabsf(g)), hh = fbits(h);
        if (ag > mg) mg = ag;
        if (hh > mh) mh = hh;
    }
    *max_g = bitsf(mg);
    *max_h = bitsf(mh);
}

void orc_base_scores_mc(const float *y, const float *w, int64_t rows, int32_t K, float *out) {
    double *cnt = (double *)malloc(sizeof(double) * (size_t)K);
    for (int32_t k = 0; k < K; ++k) cnt[k] = 1.0;                 /* +1 smoothing */
    for (int64_t i = 0; i < rows; ++i) cnt[(int32_t)y[i]] += w ? (double)w[i] : 1.0;
    double total = 0;
    for (int32_t k = 0; k < K; ++k) total += cnt[k];
    for (int32_t k = 0; k < K; ++k) out[k] = (float)log(cnt[k] / total);
    free(cnt);
}

void orc_quantize(const float *g, const float *h, int64_t rows, float mg, float mh,
                  uint32_t *ghq) {
    float gscale = mg > 0.0f ? 32767.0f / mg : 0.0f;
    float hscale = mh > 0.0f ? 127.0f / mh : 0.0f;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; ++i) {
        int qg = (int)rintf(g[i] * gscale);
        uint32_t qh = (uint32_t)rintf(h[i] * hscale);
        ghq[i] = ((uint32_t)(qg & 0xFFFF) << 16) | (qh & 0x7Fu);
    }
}

static inline int32_t q_grad(uint32_t q) { return (int32_t)(int16_t)(uint16_t)(q >> 16); }
static inline int32_t q_hess(uint32_t q) { return (int32_t)(q & 0x7Fu); }

/* ------------------------------------------------------------------------ */
/* Histograms: Shaders.swift:212-286 (per node, per feature, per bin)       */
/* ------------------------------------------------------------------------ */

void orc_hist_node(const uint8_t *bins_fm, int64_t rows, int32_t cols, int32_t nb,
                   const uint32_t *ghq, const uint32_t *row_idx, int64_t n,
                   int64_t *hg, int64_t *hh) {
    memset(hg, 0, sizeof(int64_t) * (size_t)cols * (size_t)nb);
    memset(hh, 0, sizeof(int64_t) * (size_t)cols * (size_t)nb);
    for (int64_t r = 0; r < n; ++r) {
        int64_t i = row_idx ? (int64_t)row_idx[r] : r;
        uint32_t q = ghq[i];
        int32_t qg = q_grad(q), qh = q_hess(q);
        for (int32_t f = 0; f < cols; ++f) {
            uint8_t b = bins_fm[(int64_t)f * rows + i];
            hg[(int64_t)f * nb + b] += qg;
            hh[(int64_t)f * nb + b] += qh;
        }
    }
}

/* Row-major variant used inside orc_fit (same sums, cache-friendly).  Large
 * nodes are split over threads, each with private tables that are then added
 * up: integer sums, so the result does not depend on the split. */
static void hist_rows_serial(const uint8_t *rm, int32_t cols, int32_t nb, const uint32_t *ghq,
                             const uint32_t *idx, int64_t n, int64_t *hg, int64_t *hh) {
    for (int64_t r = 0; r < n; ++r) {
        int64_t i = idx[r];
        uint32_t q = ghq[i];
        int32_t qg = q_grad(q), qh = q_hess(q);
        const uint8_t *row = rm + i * cols;
        for (int32_t f = 0; f < cols; ++f) {
            int64_t k = (int64_t)f * nb + row[f];
            hg[k] += qg;
            hh[k] += qh;
        }
    }
}

static void hist_rows_rm(const uint8_t *rm, int32_t cols, int32_t nb, const uint32_t *ghq,
                         const uint32_t *idx, int64_t n, int64_t *hg, int64_t *hh) {
    const int64_t slice = (int64_t)cols * nb;
    memset(hg, 0, sizeof(int64_t) * (size_t)slice);
    memset(hh, 0, sizeof(int64_t) * (size_t)slice);
    const int nt = omp_get_max_threads();
    if (nt <= 1 || n < 65536) {
        hist_rows_serial(rm, cols, nb, ghq, idx, n, hg, hh);
        return;
    }
    int64_t *priv = (int64_t *)calloc((size_t)nt * 2 * (size_t)slice, sizeof(int64_t));
#pragma omp parallel num_threads(nt)
    {
        const int t = omp_get_thread_num(), k = omp_get_num_threads();
        const int64_t a = n * t / k, b = n * (t + 1) / k;
        int64_t *pg = priv + (int64_t)t * 2 * slice, *ph = pg + slice;
        hist_rows_serial(rm, cols, nb, ghq, idx + a, b - a, pg, ph);
#pragma omp barrier
#pragma omp for schedule(static)
        for (int64_t j = 0; j < slice; ++j) {
            int64_t sg = 0, sh = 0;
            for (int u = 0; u < k; ++u) {
                sg += priv[(int64_t)u * 2 * slice + j];
                sh += priv[(int64_t)u * 2 * slice + slice + j];
            }
            hg[j] = sg;
            hh[j] = sh;
        }
    }
    free(priv);
}

/* ------------------------------------------------------------------------ */
/* Split search: find_splits + cat_sort, Shaders.swift:336-464              */
/* ------------------------------------------------------------------------ */

/* Non-empty bins (hess > 0) stably sorted ascending by g / (h + catSmooth):
 * the insertion sort of Shaders.swift:339-359. */
int32_t orc_cat_order(const int64_t *hg, const int64_t *hh, int32_t nb, float g_inv,
                      float h_inv, float cat_smooth, uint16_t *order) {
    float key[256];
    int32_t m = 0;
    for (int32_t b = 0; b < nb; ++b) {
        float hb = (float)hh[b] * h_inv;
        if (hb > 0.0f) {
            order[m] = (uint16_t)b;
            key[m] = ((float)hg[b] * g_inv) / (hb + cat_smooth);
            ++m;
        }
    }
    for (int32_t i = 1; i < m; ++i) {
        uint16_t ob = order[i];
        float ok = key[i];
        int32_t j = i - 1;
        while (j >= 0 && key[j] > ok) { key[j + 1] = key[j]; order[j + 1] = order[j]; --j; }
        key[j + 1] = ok;
        order[j + 1] = ob;
    }
    return m;
}

static inline float split_gain(float gl, float hl, float gr, float hr, float lambda,
                               float parent) {
    float a = (gl * gl) / (hl + lambda);
    float b = (gr * gr) / (hr + lambda);
    return (a + b) - parent;
}

void orc_find_split(const int64_t *hg, const int64_t *hh, int32_t nb, int is_cat,
                    int cst, int64_t g_tot, int64_t h_tot, float g_inv, float h_inv,
                    float lambda, float mch, float cat_smooth, orc_split *out) {
    orc_split best;
    best.gain = -INFINITY; best.bin = 0; best.gl = 0; best.hl = 0; best.flags = 0;
    best.gl_int = 0; best.hl_int = 0;
    float G = (float)g_tot * g_inv, H = (float)h_tot * h_inv;
    float parent = (G * G) / (H + lambda);
    int32_t data_bins = nb - 1;
    if (is_cat) {
        uint16_t order[256];
        int32_t m = orc_cat_order(hg, hh, nb, g_inv, h_inv, cat_smooth, order);
        int64_t GL = 0, HL = 0;
        for (int32_t i = 0; i + 1 < m; ++i) {
            int32_t b = order[i];
            GL += hg[b]; HL += hh[b];
            float gl = (float)GL * g_inv, hl = (float)HL * h_inv;
            float gr = (float)(g_tot - GL) * g_inv, hr = (float)(h_tot - HL) * h_inv;
            if (hl < mch || hr < mch) continue;
            float gain = split_gain(gl, hl, gr, hr, lambda, parent);
            if (gain > best.gain) {
                best.gain = gain; best.bin = (uint32_t)(i + 1); best.gl = gl; best.hl = hl;
                best.flags = ORC_FLAG_CATEGORICAL; best.gl_int = GL; best.hl_int = HL;
            }
        }
    } else {
        int64_t GM = hg[data_bins], HM = hh[data_bins];
        float Hm = (float)HM * h_inv;
        int64_t GL = 0, HL = 0;
        for (int32_t b = 0; b + 1 < data_bins; ++b) {
            GL += hg[b]; HL += hh[b];
            {   /* missing goes right */
                float gl = (float)GL * g_inv, hl = (float)HL * h_inv;
                float gr = (float)(g_tot - GL) * g_inv, hr = (float)(h_tot - HL) * h_inv;
                if (hl >= mch && hr >= mch) {
                    int ok = 1;
                    if (cst != 0) {
                        float vl = -gl / (hl + lambda), vr = -gr / (hr + lambda);
                        ok = cst > 0 ? vl <= vr : vl >= vr;
                    }
                    float gain = split_gain(gl, hl, gr, hr, lambda, parent);
                    if (ok && gain > best.gain) {
                        best.gain = gain; best.bin = (uint32_t)b; best.gl = gl; best.hl = hl;
                        best.flags = 0; best.gl_int = GL; best.hl_int = HL;
                    }
                }
            }
            if (Hm > 0.0f) {   /* missing goes left */
                int64_t LG = GL + GM, LH = HL + HM;
                float lg = (float)LG * g_inv, lh = (float)LH * h_inv;
                float rg = (float)(g_tot - LG) * g_inv, rh = (float)(h_tot - LH) * h_inv;
                if (lh >= mch && rh >= mch) {
                    int ok = 1;
                    if (cst != 0) {
                        float vl = -lg / (lh + lambda), vr = -rg / (rh + lambda);
                        ok = cst > 0 ? vl <= vr : vl >= vr;
                    }
                    float gain = split_gain(lg, lh, rg, rh, lambda, parent);
                    if (ok && gain > best.gain) {
                        best.gain = gain; best.bin = (uint32_t)b; best.gl = lg; best.hl = lh;
                        best.flags = ORC_FLAG_DEFAULT_LEFT; best.gl_int = LG; best.hl_int = LH;
                    }
                }
            }
        }
    }
    *out = best;
}

/* goes_left / part_left on a bin: Shaders.swift:468-476, :511-518 */
static inline int bin_goes_left(uint8_t b, uint32_t bin, uint32_t flags, const uint32_t *mask,
                                int32_t nb) {
    if (flags & ORC_FLAG_CATEGORICAL) return (int)((mask[b >> 5] >> (b & 31u)) & 1u);
    if (b == (uint8_t)(nb - 1)) return (flags & ORC_FLAG_DEFAULT_LEFT) != 0;
    return b <= (uint8_t)bin;
}

/* ------------------------------------------------------------------------ */
/* Tree growth                                                               */
/* ------------------------------------------------------------------------ */

typedef struct {
    const orc_params *p;
    const uint8_t *rm;          /* row-major bins [rows][cols] */
    const uint8_t *fm;          /* feature-major bins [cols][rows] */
    int64_t rows;
    int32_t cols, nb;
    const uint8_t *is_cat;
    const int8_t *mono;
    const float *edges;
    const uint32_t *ghq;
    float g_inv, h_inv;
    const uint32_t *rows_in;    /* the tree's rows (ascending); NULL = all rows */
    int64_t n_in;
    int apply_preds;            /* 0: preds are updated by a walk after the tree */
    float *node_lo, *node_hi;   /* out: the tree's leaf bounds per node (or NULL) */
} fit_ctx;

static void best_over_features(const fit_ctx *c, const int64_t *hg, const int64_t *hh,
                               int64_t gt, int64_t ht, const uint8_t *feat_mask,
                               int32_t *best_f, orc_split *best) {
    /* argmax over features with strict '>' (Shaders.swift:1394-1400) */
    const orc_params *p = c->p;
    *best_f = -1;
    best->gain = -INFINITY; best->bin = 0; best->gl = 0; best->hl = 0; best->flags = 0;
    best->gl_int = 0; best->hl_int = 0;
    for (int32_t f = 0; f < c->cols; ++f) {
        if (feat_mask && !feat_mask[f]) continue;   /* colsample (Shaders.swift:390-395) */
        orc_split r;
        orc_find_split(hg + (int64_t)f * c->nb, hh + (int64_t)f * c->nb, c->nb,
                       c->is_cat ? c->is_cat[f] : 0, c->mono ? c->mono[f] : 0, gt, ht,
                       c->g_inv, c->h_inv, p->lambda, p->min_child_hess, p->cat_smooth, &r);
        if (r.gain > best->gain) { *best = r; *best_f = f; }
    }
}

static void make_mask(const fit_ctx *c, const int64_t *hg, const int64_t *hh,
                      const orc_split *s, uint32_t *mask) {
    memset(mask, 0, 8 * sizeof(uint32_t));
    if (!(s->flags & ORC_FLAG_CATEGORICAL)) return;
    uint16_t order[256];
    orc_cat_order(hg, hh, c->nb, c->g_inv, c->h_inv, c->p->cat_smooth, order);
    for (uint32_t i = 0; i < s->bin; ++i) mask[order[i] >> 5] |= 1u << (order[i] & 31u);
}

static float leaf_value(const fit_ctx *c, int64_t gi, int64_t hi_, float lo, float hi) {
    float G = (float)gi * c->g_inv, H = (float)hi_ * c->h_inv;
    return c->p->learning_rate * clampf(-G / (H + c->p->lambda), lo, hi);
}

/* Monotone bound propagation (Shaders.swift:1424-1443). */
static void child_bounds(const fit_ctx *c, int32_t f, const orc_split *s, int64_t gt,
                         int64_t ht, float plo, float phi, float *llo, float *lhi,
                         float *rlo, float *rhi) {
    *llo = plo; *lhi = phi; *rlo = plo; *rhi = phi;
    int cst = (s->flags & ORC_FLAG_CATEGORICAL) ? 0 : (c->mono ? c->mono[f] : 0);
    if (cst == 0) return;
    float lambda = c->p->lambda;
    float vl = -s->gl / (s->hl + lambda);
    float gr = (float)(gt - s->gl_int) * c->g_inv, hr = (float)(ht - s->hl_int) * c->h_inv;
    float vr = -gr / (hr + lambda);
    float mid = clampf(0.5f * (vl + vr), plo, phi);
    if (cst > 0) { *lhi = fminf(*lhi, mid); *rlo = fmaxf(*rlo, mid); }
    else { *llo = fmaxf(*llo, mid); *rhi = fminf(*rhi, mid); }
}

/* Stable two-way partition of a segment by the split rule (Shaders.swift:569-620). */
static int64_t partition_stable(const fit_ctx *c, uint32_t *seg, int64_t n, int32_t f,
                                uint32_t bin, uint32_t flags, const uint32_t *mask,
                                uint32_t *tmp) {
    const uint8_t *col = c->fm + (int64_t)f * c->rows;
    int64_t nl = 0, nr = 0, left_total = 0;
    for (int64_t r = 0; r < n; ++r)
        if (bin_goes_left(col[seg[r]], bin, flags, mask, c->nb)) ++left_total;
    for (int64_t r = 0; r < n; ++r) {
        uint32_t i = seg[r];
        if (bin_goes_left(col[i], bin, flags, mask, c->nb)) tmp[nl++] = i;
        else tmp[left_total + nr++] = i;
    }
    memcpy(seg, tmp, sizeof(uint32_t) * (size_t)n);
    return left_total;
}

static void write_split(orc_forest *out, int64_t base, int32_t n, int32_t f,
                        const orc_split *s, const uint32_t *mask, const float *edges,
                        int32_t nb) {
    out->feature[base + n] = f;
    out->flags[base + n] = (uint8_t)s->flags;
    out->gain[base + n] = s->gain;
    out->leaf[base + n] = 0.0f;
    if (out->split_bin) out->split_bin[base + n] = s->bin;
    if (s->flags & ORC_FLAG_CATEGORICAL) {
        out->threshold[base + n] = 0.0f;
        if (out->cat_mask) memcpy(out->cat_mask + (base + n) * 8, mask, 8 * sizeof(uint32_t));
    } else {
        out->threshold[base + n] = edges[(int64_t)f * (nb - 2) + s->bin];
    }
}

/* Level-wise growth: init_tree/decide_splits/route_samples/final_leaves
 * (Shaders.swift:1317-1511, Booster.swift:1321-1648). */
static int grow_levelwise(const fit_ctx *c, float *preds, orc_forest *out, int64_t base,
                          const uint8_t *feat_mask) {
    const orc_params *p = c->p;
    int32_t D = p->max_depth, F = c->cols, nb = c->nb;
    int32_t total = (1 << (D + 1)) - 1;
    int64_t slice = (int64_t)F * nb;
    int64_t N = c->rows;
    int64_t *cnt = (int64_t *)calloc((size_t)total, sizeof(int64_t));
    int64_t *seg = (int64_t *)calloc((size_t)total, sizeof(int64_t));
    int64_t *gi = (int64_t *)calloc((size_t)total, sizeof(int64_t));
    int64_t *hi = (int64_t *)calloc((size_t)total, sizeof(int64_t));
    float *blo = (float *)malloc(sizeof(float) * (size_t)total);
    float *bhi = (float *)malloc(sizeof(float) * (size_t)total);
    int32_t max_level = 1 << (D - 1);
    int64_t *cur_g = (int64_t *)malloc(sizeof(int64_t) * (size_t)(slice * max_level));
    int64_t *cur_h = (int64_t *)malloc(sizeof(int64_t) * (size_t)(slice * max_level));
    int64_t *prv_g = (int64_t *)malloc(sizeof(int64_t) * (size_t)(slice * max_level));
    int64_t *prv_h = (int64_t *)malloc(sizeof(int64_t) * (size_t)(slice * max_level));
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)N);
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)N);
    if (!cnt || !seg || !gi || !hi || !blo || !bhi || !cur_g || !cur_h || !prv_g || !prv_h ||
        !order || !tmp) {
        free(cnt); free(seg); free(gi); free(hi); free(blo); free(bhi); free(cur_g);
        free(cur_h); free(prv_g); free(prv_h); free(order); free(tmp);
        return -1;
    }
    for (int32_t n = 0; n < total; ++n) { blo[n] = -INFINITY; bhi[n] = INFINITY; }
    if (c->rows_in) {
        memcpy(order, c->rows_in, sizeof(uint32_t) * (size_t)c->n_in);
        N = c->n_in;
    } else {
        for (int64_t i = 0; i < N; ++i) order[i] = (uint32_t)i;
    }
    cnt[0] = N; seg[0] = 0;
    int32_t *split_f = (int32_t *)malloc(sizeof(int32_t) * (size_t)total);
    for (int32_t n = 0; n < total; ++n) split_f[n] = -1;

    for (int32_t d = 0; d < D; ++d) {
        int32_t ls = (1 << d) - 1, nl = 1 << d;
        /* histograms: smaller sibling built, larger derived (Shaders.swift:1466-1479) */
        if (d == 0) {
            hist_rows_rm(c->rm, F, nb, c->ghq, order, N, cur_g, cur_h);
            int64_t G = 0, H = 0;
            for (int32_t b = 0; b < nb; ++b) { G += cur_g[b]; H += cur_h[b]; }
            gi[0] = G; hi[0] = H;
        } else {
            for (int32_t local = 0; local < nl; local += 2) {
                int32_t l = ls + local, r = l + 1, par = (l - 1) / 2;
                if (split_f[par] < 0) continue;
                int32_t plocal = par - ((1 << (d - 1)) - 1);
                int built = cnt[l] <= cnt[r] ? l : r;
                int derived = built == l ? r : l;
                int64_t *bg = cur_g + (int64_t)(built - ls) * slice;
                int64_t *bh = cur_h + (int64_t)(built - ls) * slice;
                int64_t *dg = cur_g + (int64_t)(derived - ls) * slice;
                int64_t *dh = cur_h + (int64_t)(derived - ls) * slice;
                hist_rows_rm(c->rm, F, nb, c->ghq, order + seg[built], cnt[built], bg, bh);
                const int64_t *pg = prv_g + (int64_t)plocal * slice;
                const int64_t *ph = prv_h + (int64_t)plocal * slice;
                for (int64_t k = 0; k < slice; ++k) { dg[k] = pg[k] - bg[k]; dh[k] = ph[k] - bh[k]; }
            }
        }
        /* decisions (decide_splits, Shaders.swift:1386-1451) */
        int64_t next_start = 0;
        for (int32_t local = 0; local < nl; ++local) {
            int32_t n = ls + local;
            int32_t lc = 2 * n + 1, rc = 2 * n + 2;
            if (cnt[n] < 1) {
                out->feature[base + n] = -1;
                out->leaf[base + n] = 0.0f;
                out->gain[base + n] = 0.0f;
                continue;
            }
            const int64_t *hg = cur_g + (int64_t)local * slice;
            const int64_t *hh = cur_h + (int64_t)local * slice;
            int32_t bf;
            orc_split best;
            best_over_features(c, hg, hh, gi[n], hi[n], feat_mask, &bf, &best);
            if (bf >= 0 && isfinite(best.gain) && best.gain > p->min_split_gain) {
                uint32_t mask[8];
                make_mask(c, hg + (int64_t)bf * nb, hh + (int64_t)bf * nb, &best, mask);
                write_split(out, base, n, bf, &best, mask, c->edges, nb);
                split_f[n] = bf;
                gi[lc] = best.gl_int; hi[lc] = best.hl_int;
                gi[rc] = gi[n] - best.gl_int; hi[rc] = hi[n] - best.hl_int;
                child_bounds(c, bf, &best, gi[n], hi[n], blo[n], bhi[n], &blo[lc], &bhi[lc],
                             &blo[rc], &bhi[rc]);
                int64_t left = partition_stable(c, order + seg[n], cnt[n], bf, best.bin,
                                                best.flags, mask, tmp);
                cnt[lc] = left; cnt[rc] = cnt[n] - left;
            } else {
                float v = leaf_value(c, gi[n], hi[n], blo[n], bhi[n]);
                out->feature[base + n] = -1;
                out->leaf[base + n] = v;
                out->gain[base + n] = 0.0f;
                if (c->apply_preds)
                    for (int64_t r = 0; r < cnt[n]; ++r) preds[order[seg[n] + r]] += v;
            }
        }
        /* Next level's segment layout: children in heap order, every split
         * parent contributing [left | right] (partition_stable already
         * ordered its segment that way); rows of new leaves leave the active
         * set (Shaders.swift:1455-1480, :1280-1281).  Moving segments left
         * in heap order never overwrites an unmoved segment. */
        {
            int64_t pos = 0;
            for (int32_t local = 0; local < nl; ++local) {
                int32_t n = ls + local, lc = 2 * n + 1, rc = 2 * n + 2;
                if (split_f[n] < 0 || cnt[n] < 1) {
                    cnt[lc] = 0; cnt[rc] = 0;
                    seg[lc] = next_start; seg[rc] = next_start;
                    continue;
                }
                if (seg[n] != pos)
                    memmove(order + pos, order + seg[n], sizeof(uint32_t) * (size_t)cnt[n]);
                seg[lc] = pos;
                seg[rc] = pos + cnt[lc];
                pos += cnt[n];
                next_start = pos;
            }
        }
        int64_t *sw;
        sw = cur_g; cur_g = prv_g; prv_g = sw;
        sw = cur_h; cur_h = prv_h; prv_h = sw;
    }
    /* deepest level: every node is a leaf (final_leaves, Shaders.swift:1495-1511) */
    {
        int32_t ls = (1 << D) - 1, nl = 1 << D;
        for (int32_t local = 0; local < nl; ++local) {
            int32_t n = ls + local;
            out->feature[base + n] = -1;
            out->gain[base + n] = 0.0f;
            if (cnt[n] >= 1) {
                float v = leaf_value(c, gi[n], hi[n], blo[n], bhi[n]);
                out->leaf[base + n] = v;
                if (c->apply_preds)
                    for (int64_t r = 0; r < cnt[n]; ++r) preds[order[seg[n] + r]] += v;
            } else {
                out->leaf[base + n] = 0.0f;
            }
        }
    }
    for (int32_t n = 0; n < total; ++n) out->cover[base + n] = (float)cnt[n];
    free(split_f);
    if (c->node_lo) {
        memcpy(c->node_lo, blo, sizeof(float) * (size_t)total);
        memcpy(c->node_hi, bhi, sizeof(float) * (size_t)total);
    }
    free(cnt); free(seg); free(gi); free(hi); free(blo); free(bhi); free(cur_g);
    free(cur_h); free(prv_g); free(prv_h); free(order); free(tmp);
    return 0;
}

/* Train preds: one walk of the finished tree over every binned row
 * (predict_tree_binned, Shaders.swift:1763-1781). */
static void walk_preds(const fit_ctx *c, const orc_forest *out, int64_t base, float *preds) {
    const int32_t D = c->p->max_depth, nb = c->nb;
    const int64_t N = c->rows;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        int32_t n = 0;
        for (int32_t d = 0; d < D; ++d) {
            int32_t f = out->feature[base + n];
            if (f < 0) break;
            uint8_t b = c->fm[(int64_t)f * N + i];
            const uint32_t *mask = out->cat_mask ? out->cat_mask + (base + n) * 8 : NULL;
            uint32_t zero[8] = {0};
            n = 2 * n + 1 + (bin_goes_left(b, out->split_bin[base + n], out->flags[base + n],
                                           mask ? mask : zero, nb) ? 0 : 1);
        }
        preds[i] += out->leaf[base + n];
    }
}

/* Leaf-wise (best-first) growth: leaf_reset/leaf_init/leaf_pick_apply and the
 * partition pipeline (Shaders.swift:656-1091, Booster.swift:967-1310). */
typedef struct {
    int32_t node;
    int64_t seg, count, G, H;
    int32_t depth, best_f;
    orc_split best;
} lw_open;

static int grow_leafwise(const fit_ctx *c, float *preds, orc_forest *out, int64_t base,
                         const uint8_t *feat_mask) {
    const orc_params *p = c->p;
    int32_t D = p->max_depth, F = c->cols, nb = c->nb, L = p->num_leaves;
    int32_t total = (1 << (D + 1)) - 1;
    int64_t slice = (int64_t)F * nb, N = c->rows;
    const int64_t n_tree = c->rows_in ? c->n_in : N;
    float *blo = (float *)malloc(sizeof(float) * (size_t)total);
    float *bhi = (float *)malloc(sizeof(float) * (size_t)total);
    lw_open *open = (lw_open *)calloc((size_t)(2 * L + 2), sizeof(lw_open));
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)N);
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)N);
    int64_t *hg = (int64_t *)malloc(sizeof(int64_t) * (size_t)slice);
    int64_t *hh = (int64_t *)malloc(sizeof(int64_t) * (size_t)slice);
    if (!blo || !bhi || !open || !order || !tmp || !hg || !hh) {
        free(blo); free(bhi); free(open); free(order); free(tmp); free(hg); free(hh);
        return -1;
    }
    for (int32_t n = 0; n < total; ++n) {
        out->feature[base + n] = -1; out->leaf[base + n] = 0; out->gain[base + n] = 0;
        out->cover[base + n] = 0; out->threshold[base + n] = 0; out->flags[base + n] = 0;
        if (out->split_bin) out->split_bin[base + n] = 0;
        if (out->cat_mask) memset(out->cat_mask + (base + n) * 8, 0, 32);
        blo[n] = -FLT_MAX; bhi[n] = FLT_MAX;
    }
    if (c->rows_in) memcpy(order, c->rows_in, sizeof(uint32_t) * (size_t)n_tree);
    else for (int64_t i = 0; i < N; ++i) order[i] = (uint32_t)i;
    /* leaf_init (Shaders.swift:683-716) */
    hist_rows_rm(c->rm, F, nb, c->ghq, order, n_tree, hg, hh);
    int64_t G0 = 0, H0 = 0;
    for (int32_t b = 0; b < nb; ++b) { G0 += hg[b]; H0 += hh[b]; }
    open[0].node = 0; open[0].seg = 0; open[0].count = n_tree; open[0].G = G0; open[0].H = H0;
    open[0].depth = 0;
    best_over_features(c, hg, hh, G0, H0, feat_mask, &open[0].best_f, &open[0].best);
    out->leaf[base + 0] = leaf_value(c, G0, H0, -FLT_MAX, FLT_MAX);
    out->cover[base + 0] = (float)n_tree;
    int32_t open_count = 1, leaves = 1, done = 0;
    for (int32_t it = 1; it < L; ++it) {
        if (done || leaves >= L) { done = 1; continue; }
        int32_t bi = -1;
        float bg = p->min_split_gain;
        for (int32_t i = 0; i < open_count; ++i)
            if (open[i].best_f >= 0 && isfinite(open[i].best.gain) && open[i].best.gain > bg) {
                bg = open[i].best.gain; bi = i;
                if (p->plant == ORC_PLANT_FIFO_PICK) break;
            }
        if (bi < 0) { done = 1; continue; }
        lw_open Lp = open[bi];
        int32_t bf = Lp.best_f;
        orc_split best = Lp.best;
        /* parent histogram, needed only to rebuild a categorical subset mask */
        if (best.flags & ORC_FLAG_CATEGORICAL)
            hist_rows_rm(c->rm, F, nb, c->ghq, order + Lp.seg, Lp.count, hg, hh);
        uint32_t mask[8];
        make_mask(c, hg + (int64_t)bf * nb, hh + (int64_t)bf * nb, &best, mask);
        write_split(out, base, Lp.node, bf, &best, mask, c->edges, nb);
        int64_t lcount = partition_stable(c, order + Lp.seg, Lp.count, bf, best.bin,
                                          best.flags, mask, tmp);
        int64_t rcount = Lp.count - lcount;
        int32_t lc = 2 * Lp.node + 1, rc = 2 * Lp.node + 2;
        int64_t lG = best.gl_int, lH = best.hl_int, rG = Lp.G - lG, rH = Lp.H - lH;
        child_bounds(c, bf, &best, Lp.G, Lp.H, blo[Lp.node], bhi[Lp.node], &blo[lc], &bhi[lc],
                     &blo[rc], &bhi[rc]);
        out->cover[base + lc] = (float)lcount;
        out->cover[base + rc] = (float)rcount;
        out->leaf[base + lc] = leaf_value(c, lG, lH, blo[lc], bhi[lc]);
        out->leaf[base + rc] = leaf_value(c, rG, rH, blo[rc], bhi[rc]);
        int32_t child_depth = Lp.depth + 1;
        int can_eval = child_depth < D && leaves + 1 < L && lcount > 0 && rcount > 0;
        int32_t i0 = open_count, i1 = open_count + 1;
        open_count += 2;
        leaves += 1;
        open[bi].best_f = -1;
        open[bi].best.gain = -INFINITY;
        lw_open cl, cr;
        memset(&cl, 0, sizeof cl);
        cl.node = lc; cl.seg = Lp.seg; cl.count = lcount; cl.G = lG; cl.H = lH;
        cl.depth = child_depth; cl.best_f = -1; cl.best.gain = -INFINITY;
        cr = cl;
        cr.node = rc; cr.seg = Lp.seg + lcount; cr.count = rcount; cr.G = rG; cr.H = rH;
        if (can_eval) {
            lw_open *ch[2] = {&cl, &cr};
            for (int k = 0; k < 2; ++k) {
                lw_open *o = ch[k];
                hist_rows_rm(c->rm, F, nb, c->ghq, order + o->seg, o->count, hg, hh);
                best_over_features(c, hg, hh, o->G, o->H, feat_mask, &o->best_f, &o->best);
            }
        }
        open[i0] = cl;
        open[i1] = cr;
    }
    walk_preds(c, out, base, preds);
    if (c->node_lo) {
        memcpy(c->node_lo, blo, sizeof(float) * (size_t)total);
        memcpy(c->node_hi, bhi, sizeof(float) * (size_t)total);
    }
    free(blo); free(bhi); free(open); free(order); free(tmp); free(hg); free(hh);
    return 0;
}

/* The leaf a binned row reaches (assign_leaves). */
static int32_t leaf_of_row(const fit_ctx *c, const orc_forest *out, int64_t base, int64_t i) {
    const int32_t D = c->p->max_depth, nb = c->nb;
    static const uint32_t zero[8] = {0};
    int32_t n = 0;
    for (int32_t d = 0; d < D; ++d) {
        int32_t f = out->feature[base + n];
        if (f < 0) break;
        uint8_t b = c->fm[(int64_t)f * c->rows + i];
        const uint32_t *mask = out->cat_mask ? out->cat_mask + (base + n) * 8 : zero;
        n = 2 * n + 1 + (bin_goes_left(b, out->split_bin[base + n], out->flags[base + n], mask,
                                       nb) ? 0 : 1);
    }
    return n;
}

/* Leaf renewal for the L1 and quantile objectives (Booster.swift:634-639,
 * :1596-1615 level-wise, :1253-1290 leaf-wise): residuals y - preds over
 * the rows i = 0, step, 2*step, ... (step = max(1, rows/262144)), bucketed by
 * the row's leaf; a leaf with >= 4 sampled residuals becomes
 * lr * min(max(r[min(n-1, (int)((float)n*q))], lo), hi) over the sorted r.
 * With delta != NULL (leaf-wise: preds already hold the tree's first leaf
 * values) a changed leaf records delta[n] = new - old, else delta[n] = 0. */
static void renew_leaves(const fit_ctx *c, orc_forest *out, int64_t base, const float *y,
                         const float *preds, float q, float *delta) {
    const int32_t total = out->nodes_per_tree;
    const int64_t N = c->rows;
    int64_t step = N / 262144;
    if (step < 1) step = 1;
    const int64_t ns = (N + step - 1) / step;
    int32_t *leaf = (int32_t *)malloc(sizeof(int32_t) * (size_t)ns);
    int64_t *cnt = (int64_t *)calloc((size_t)total + 1, sizeof(int64_t));
    float *res = (float *)malloc(sizeof(float) * (size_t)ns);
    int64_t *pos = (int64_t *)malloc(sizeof(int64_t) * ((size_t)total + 1));
    for (int64_t s = 0; s < ns; ++s) {
        leaf[s] = leaf_of_row(c, out, base, s * step);
        cnt[leaf[s]]++;
    }
    int64_t acc = 0;
    for (int32_t n = 0; n < total; ++n) { pos[n] = acc; acc += cnt[n]; }
    int64_t *fill = (int64_t *)malloc(sizeof(int64_t) * (size_t)total);
    memcpy(fill, pos, sizeof(int64_t) * (size_t)total);
    for (int64_t s = 0; s < ns; ++s) {
        int64_t i = s * step;
        res[fill[leaf[s]]++] = y[i] - preds[i];
    }
    for (int32_t n = 0; n < total; ++n) {
        if (delta) delta[n] = 0.0f;
        if (cnt[n] < 4) continue;
        float *r = res + pos[n];
        qsort(r, (size_t)cnt[n], sizeof(float), cmp_float);
        int64_t k = (int64_t)((float)cnt[n] * q);
        if (k > cnt[n] - 1) k = cnt[n] - 1;
        float v = r[k];
        v = v > c->node_lo[n] ? v : c->node_lo[n];
        v = v < c->node_hi[n] ? v : c->node_hi[n];
        v = c->p->learning_rate * v;
        if (delta) {
            if (v != out->leaf[base + n]) {
                delta[n] = v - out->leaf[base + n];
                out->leaf[base + n] = v;
            }
        } else {
            out->leaf[base + n] = v;
        }
    }
    free(leaf); free(cnt); free(res); free(pos); free(fill);
}

/* ------------------------------------------------------------------------ */
/* Row sampling: GOSS and bagging                                           */
/* ------------------------------------------------------------------------ */

/* gossActive / bagging (Booster.swift:1382-1384): GOSS after ceil(1/lr)
 * warm-up trees, bagging on every tree. */
int orc_sampling_active(const orc_params *p, int32_t tree) {
    if (p->goss) return tree >= (int32_t)ceilf(1.0f / p->learning_rate);
    return p->subsample < 1.0f;
}

static inline uint32_t wang_hash(uint32_t x) {                    /* :1144-1148 */
    x = (x ^ 61u) ^ (x >> 16);
    x *= 9u;
    x ^= x >> 4;
    x *= 0x27d4eb2du;
    x ^= x >> 15;
    return x;
}

/* Boruta shadows (shadow_perm + shadow_bins, Shaders.swift:1596-1631): a
 * 4-round Feistel permutation of [0, n) over 2*hb bits with cycle walking;
 * fm2 [2*cols][rows] holds the real bins, then column f's bins permuted by
 * the round seed ^ wang_hash(f + 1). */
uint32_t orc_shadow_perm(uint32_t i, uint32_t n, uint32_t hb, uint32_t seed) {
    const uint32_t mask = (1u << hb) - 1u;
    do {
        uint32_t L = i >> hb, R = i & mask;
        for (uint32_t r = 0; r < 4; ++r) {
            uint32_t t = R;
            R = L ^ (wang_hash(R ^ (seed + r * 0x9E3779B9u)) & mask);
            L = t;
        }
        i = (L << hb) | R;
    } while (i >= n);
    return i;
}

void orc_shadow_bins(const uint8_t *fm, int64_t rows, int32_t cols, uint32_t hb, uint32_t seed,
                     uint8_t *fm2) {
    for (int32_t f = 0; f < cols; ++f) {
        const uint32_t fs = seed ^ wang_hash((uint32_t)f + 1u);
        for (int64_t i = 0; i < rows; ++i) {
            fm2[(int64_t)f * rows + i] = fm[(int64_t)f * rows + i];
            const uint32_t j = orc_shadow_perm((uint32_t)i, (uint32_t)rows, hb, fs);
            fm2[(int64_t)(cols + f) * rows + i] = fm[(int64_t)f * rows + j];
        }
    }
}

int64_t orc_sample_rows(const orc_params *p, int32_t tree, float *g, float *h, int64_t rows,
                        float max_g, uint8_t *kept, float *wmax_g, float *wmax_h) {
    const int goss = p->goss != 0;
    /* keep threshold: lower edge of the |g| bucket where the count from the
     * top reaches topCount (goss_grad_hist / goss_threshold, :1104-1138);
     * bagging uses topCount = 0, i.e. the threshold max|g| */
    uint32_t b = 1024;
    if (goss && max_g > 0.0f) {
        uint32_t buckets[1024] = {0};
        for (int64_t i = 0; i < rows; ++i) {
            uint32_t k = (uint32_t)(fabsf(g[i]) / max_g * 1024.0f);
            buckets[k < 1023u ? k : 1023u] += 1;
        }
        const uint32_t top = (uint32_t)((float)rows * p->goss_top_rate);
        uint32_t cum = 0;
        while (b > 0 && cum < top) { b -= 1; cum += buckets[b]; }
    }
    const float thr = max_g > 0.0f ? (float)b / 1024.0f * max_g : 0.0f;
    const float other = goss ? p->goss_other_rate / (1.0f - p->goss_top_rate) : p->subsample;
    const float weight = goss ? (1.0f - p->goss_top_rate) / p->goss_other_rate : 1.0f;
    const uint32_t seed = (uint32_t)tree + 1u;
    /* keep the top rows, and a hashed uniform sample of the rest amplified by
     * `weight` (goss_select, :1150-1199) */
    uint32_t mgb = 0, mhb = 0;
    int64_t n = 0;
    for (int64_t i = 0; i < rows; ++i) {
        const float ag = fabsf(g[i]);
        int keep = 0;
        float w = 1.0f;
        if (ag >= thr) {
            keep = 1;
        } else {
            const uint32_t hv = p->plant == ORC_PLANT_GOSS_NO_SEED
                                    ? wang_hash((uint32_t)i)
                                    : wang_hash((uint32_t)i ^ (seed * 0x9E3779B9u));
            if ((float)(hv >> 8) * (1.0f / 16777216.0f) < other) { keep = 1; w = weight; }
        }
        const float hw = h[i] * w;
        kept[i] = (uint8_t)keep;
        if (!keep) continue;
        if (w != 1.0f) { g[i] = g[i] * w; h[i] = hw; }
        const float agw = ag * w;
        uint32_t u;
        memcpy(&u, &agw, 4); if (u > mgb) mgb = u;
        memcpy(&u, &hw, 4); if (u > mhb) mhb = u;
        ++n;
    }
    memcpy(wmax_g, &mgb, 4);
    memcpy(wmax_h, &mhb, 4);
    return n;
}

/* Per-tree feature mask (Booster.swift:684-700, :1386-1400): the allowed
 * features, each kept with probability featureFraction by a SplitMix64
 * stream seeded 0xC0150001 + t * golden (the uniform is drawn only for an
 * allowed feature); if none is kept, one allowed feature is drawn with the
 * stream's next word.  Returns 0 when every feature may split. */
static int tree_feature_mask(const orc_params *p, int32_t t, int32_t cols, uint8_t *m) {
    if (!p->allowed && !(p->feature_fraction < 1.0f)) return 0;
    int32_t n_allowed = 0;
    for (int32_t f = 0; f < cols; ++f) n_allowed += p->allowed ? p->allowed[f] != 0 : 1;
    if (!(p->feature_fraction < 1.0f)) {
        for (int32_t f = 0; f < cols; ++f) m[f] = p->allowed ? p->allowed[f] != 0 : 1;
        return 1;
    }
    uint64_t s = 0xC0150001ULL + (uint64_t)t * GOLDEN;
    int any = 0;
    for (int32_t f = 0; f < cols; ++f) {
        const int base = p->allowed ? p->allowed[f] != 0 : 1;
        m[f] = (uint8_t)(base && orc_splitmix_uniform(&s) < p->feature_fraction);
        any |= m[f];
    }
    if (!any && n_allowed > 0) {
        int64_t k = (int64_t)(orc_splitmix_next(&s) % (uint64_t)n_allowed);
        for (int32_t f = 0; f < cols; ++f) {
            if (p->allowed && !p->allowed[f]) continue;
            if (k-- == 0) { m[f] = 1; break; }
        }
    }
    return 1;
}

int orc_fit(const orc_params *p, const uint8_t *bins_fm, int64_t rows, int32_t cols,
            const float *y, const float *w, const uint8_t *is_cat, const int8_t *monotone,
            const float *edges, float base_score, float *preds, orc_forest *out) {
    (void)base_score;
    int32_t D = p->max_depth, nb = p->num_bins;
    int32_t total = (1 << (D + 1)) - 1;
    if (out->nodes_per_tree != total) return -2;
    uint8_t *rm = (uint8_t *)malloc((size_t)rows * (size_t)cols);
    float *g = (float *)malloc(sizeof(float) * (size_t)rows);
    float *h = (float *)malloc(sizeof(float) * (size_t)rows);
    uint32_t *ghq = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)rows);
    uint8_t *kept = (uint8_t *)malloc((size_t)rows);
    uint32_t *sel = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)rows);
    float *node_lo = (float *)malloc(sizeof(float) * (size_t)total);
    float *node_hi = (float *)malloc(sizeof(float) * (size_t)total);
    float *delta = (float *)malloc(sizeof(float) * (size_t)total);
    uint8_t *fmask = (uint8_t *)malloc((size_t)cols);
    uint32_t *split_bin = out->split_bin;
    if (!rm || !g || !h || !ghq || !kept || !sel || !node_lo || !node_hi || !delta || !fmask) {
        free(rm); free(g); free(h); free(ghq); free(kept); free(sel);
        free(node_lo); free(node_hi); free(delta); free(fmask);
        return -1;
    }
#pragma omp parallel for schedule(static)
    for (int64_t i0 = 0; i0 < rows; i0 += 4096) {
        const int64_t i1 = i0 + 4096 < rows ? i0 + 4096 : rows;
        for (int32_t f = 0; f < cols; ++f)
            for (int64_t i = i0; i < i1; ++i) rm[i * cols + f] = bins_fm[(int64_t)f * rows + i];
    }
    if (!split_bin) out->split_bin = (uint32_t *)calloc((size_t)out->num_trees * total, 4);
    int rc = 0;
    const int32_t K = p->num_classes > 1 ? p->num_classes : 1;
    if (out->num_trees < p->num_trees * K) rc = -2;
    for (int32_t t = 0; t < p->num_trees * K && rc == 0; ++t) {
        int64_t base = (int64_t)t * total;
        const int32_t cls = t % K;
        float *pc = preds + (int64_t)cls * rows;     /* this tree's class */
        for (int32_t n = 0; n < total; ++n) {
            out->feature[base + n] = -1; out->threshold[base + n] = 0; out->leaf[base + n] = 0;
            out->flags[base + n] = 0; out->gain[base + n] = 0; out->cover[base + n] = 0;
            out->split_bin[base + n] = 0;
            if (out->cat_mask) memset(out->cat_mask + (base + n) * 8, 0, 32);
        }
        float mg, mh;
        if (K > 1) orc_gradients_mc(preds, y, w, rows, K, cls, g, h, &mg, &mh);
        else orc_gradients(preds, y, w, rows, p->objective, p->alpha, p->aux, g, h, &mg, &mh);
        const uint32_t *rows_in = NULL;
        int64_t n_in = rows;
        if (orc_sampling_active(p, t)) {
            /* the tree is built from the kept rows only (Booster.swift:1401-1445) */
            float wg, wh;
            n_in = orc_sample_rows(p, t, g, h, rows, mg, kept, &wg, &wh);
            mg = wg; mh = wh;
            int64_t k2 = 0;
            for (int64_t i = 0; i < rows; ++i)
                if (kept[i]) sel[k2++] = (uint32_t)i;
            rows_in = sel;
        }
        orc_quantize(g, h, rows, mg, mh, ghq);
        fit_ctx c;
        c.p = p; c.rm = rm; c.fm = bins_fm; c.rows = rows; c.cols = cols; c.nb = nb;
        c.is_cat = is_cat; c.mono = monotone; c.edges = edges; c.ghq = ghq;
        c.g_inv = mg / 32767.0f;
        c.h_inv = mh / 127.0f;
        c.rows_in = rows_in;
        c.n_in = n_in;
        const int renewal = p->objective == ORC_OBJ_MAE || p->objective == ORC_OBJ_QUANTILE;
        c.apply_preds = rows_in == NULL && !renewal;
        c.node_lo = renewal ? node_lo : NULL;
        c.node_hi = renewal ? node_hi : NULL;
        const uint8_t *tm = tree_feature_mask(p, t, cols, fmask) ? fmask : NULL;
        rc = p->num_leaves > 0 ? grow_leafwise(&c, pc, out, base, tm)
                               : grow_levelwise(&c, pc, out, base, tm);
        if (rc == 0 && renewal) {
            const float q = p->objective == ORC_OBJ_MAE ? 0.5f : p->alpha;
            if (p->num_leaves > 0) {
                /* leaf-wise: residuals after the tree's first leaf values,
                 * then the changes are added (Booster.swift:1253-1290) */
                renew_leaves(&c, out, base, y, pc, q, delta);
                for (int64_t i = 0; i < rows; ++i) pc[i] += delta[leaf_of_row(&c, out, base, i)];
            } else {
                /* level-wise: residuals before the tree (route apply = 0),
                 * then one walk with the renewed leaves (:1596-1630) */
                renew_leaves(&c, out, base, y, pc, q, NULL);
                walk_preds(&c, out, base, pc);
            }
        } else if (rc == 0 && rows_in && p->num_leaves <= 0) {
            /* sampled level-wise trees: every row's prediction from one walk
             * (Booster.swift:1568-1580); leaf-wise growth always walks */
            walk_preds(&c, out, base, pc);
        }
        /* reachable nodes only (Booster.swift:918-945) */
        {
            uint8_t *reach = (uint8_t *)calloc((size_t)total, 1);
            reach[0] = 1;
            for (int32_t n = 0; n < total; ++n) {
                if (!reach[n]) continue;
                if (out->feature[base + n] >= 0 && 2 * n + 2 < total) {
                    reach[2 * n + 1] = 1; reach[2 * n + 2] = 1;
                }
            }
            for (int32_t n = 0; n < total; ++n) {
                if (reach[n]) {
                    if (out->feature[base + n] >= 0) out->leaf[base + n] = 0.0f;
                    else {
                        out->threshold[base + n] = 0; out->flags[base + n] = 0;
                        out->gain[base + n] = 0; out->split_bin[base + n] = 0;
                        if (out->cat_mask) memset(out->cat_mask + (base + n) * 8, 0, 32);
                    }
                    continue;
                }
                out->feature[base + n] = -1; out->threshold[base + n] = 0;
                out->leaf[base + n] = 0; out->flags[base + n] = 0; out->gain[base + n] = 0;
                out->cover[base + n] = 0; out->split_bin[base + n] = 0;
                if (out->cat_mask) memset(out->cat_mask + (base + n) * 8, 0, 32);
            }
            free(reach);
        }
    }
    if (!split_bin) { free(out->split_bin); out->split_bin = NULL; }
    free(rm); free(g); free(h); free(ghq); free(kept); free(sel);
    free(node_lo); free(node_hi); free(delta); free(fmask);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Raw-feature inference: predictCPU (Booster.swift:2035-2074)              */
/* ------------------------------------------------------------------------ */

static inline int raw_goes_left(const orc_forest *m, int64_t k, float v, int32_t data_bins) {
    uint32_t fl = m->flags[k];
    if (fl & ORC_FLAG_CATEGORICAL) {
        int32_t cat = data_bins;
        if (isfinite(v)) {
            float r = rintf(v);
            if (r >= 0.0f && (int64_t)r < data_bins) cat = (int32_t)r;
        }
        return m->cat_mask ? (int)((m->cat_mask[k * 8 + cat / 32] >> (cat % 32)) & 1u) : 0;
    }
    if (isnan(v)) return (fl & ORC_FLAG_DEFAULT_LEFT) != 0;
    return v <= m->threshold[k];
}

void orc_predict(const orc_forest *m, float base, int32_t data_bins, const float *x,
                 int64_t rows, int32_t cols, float *out) {
    (void)cols;
    /* rows in chunks of 16,384 over the host cores (Booster.swift:2041-2045) */
#pragma omp parallel for schedule(dynamic, 16384)
    for (int64_t i = 0; i < rows; ++i) {
        float acc = base;
        for (int32_t t = 0; t < m->num_trees; ++t) {
            int64_t b = (int64_t)t * m->nodes_per_tree;
            int32_t n = 0;
            while (m->feature[b + n] >= 0) {
                int32_t f = m->feature[b + n];
                float v = x[(int64_t)f * rows + i];
                n = 2 * n + 1 + (raw_goes_left(m, b + n, v, data_bins) ? 0 : 1);
            }
            acc += m->leaf[b + n];
        }
        out[i] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* TreeSHAP: recursive, double precision (SHAP.swift:170-325)               */
/* ------------------------------------------------------------------------ */

typedef struct { int32_t fi; double z, o, w; } pe_t;
#define ORC_SHAP_MAXP 32

static int extend_path(pe_t *m, int len, double z, double o, int32_t fi) {  /* :266-279 */
    int l = len;
    m[l].fi = fi; m[l].z = z; m[l].o = o; m[l].w = l == 0 ? 1.0 : 0.0;
    for (int i = l - 1; i >= 0; --i) {
        m[i + 1].w += o * m[i].w * (double)(i + 1) / (double)(l + 1);
        m[i].w = z * m[i].w * (double)(l - i) / (double)(l + 1);
    }
    return l + 1;
}

static int unwind_path(pe_t *m, int len, int idx) {                       /* :281-305 */
    int l = len - 1;
    double one = m[idx].o, zero = m[idx].z, next = m[l].w;
    if (one != 0) {
        for (int i = l - 1; i >= 0; --i) {
            double tmp = m[i].w;
            m[i].w = next * (double)(l + 1) / ((double)(i + 1) * one);
            next = tmp - m[i].w * zero * (double)(l - i) / (double)(l + 1);
        }
    } else {
        for (int i = l - 1; i >= 0; --i)
            m[i].w = m[i].w * (double)(l + 1) / (zero * (double)(l - i));
    }
    for (int i = idx; i < l; ++i) { m[i].fi = m[i + 1].fi; m[i].z = m[i + 1].z; m[i].o = m[i + 1].o; }
    return l;
}

static double unwound_sum(const pe_t *m, int len, int idx) {               /* :307-325 */
    int l = len - 1;
    double one = m[idx].o, zero = m[idx].z, next = m[l].w, total = 0;
    if (one != 0) {
        for (int i = l - 1; i >= 0; --i) {
            double tmp = next / ((double)(i + 1) * one);
            total += tmp;
            next = m[i].w - tmp * zero * (double)(l - i);
        }
    } else if (zero != 0) {
        for (int i = l - 1; i >= 0; --i) total += m[i].w / (zero * (double)(l - i));
    }
    return total * (double)(l + 1);
}

static void shap_recurse(const orc_forest *mdl, int64_t tb, int32_t node, const pe_t *path,
                         int plen, double pz, double po, int32_t pf, const float *x,
                         int64_t i, int64_t rows, int32_t data_bins, double *phi) {  /* :225-264 */
    pe_t m[ORC_SHAP_MAXP];
    memcpy(m, path, sizeof(pe_t) * (size_t)plen);
    int len = extend_path(m, plen, pz, po, pf);
    if (mdl->feature[tb + node] < 0) {
        double v = (double)mdl->leaf[tb + node];
        for (int k = 1; k < len; ++k) {
            double w = unwound_sum(m, len, k);
            phi[m[k].fi] += w * (m[k].o - m[k].z) * v;
        }
        return;
    }
    int32_t f = mdl->feature[tb + node];
    int left = raw_goes_left(mdl, tb + node, x[(int64_t)f * rows + i], data_bins);
    int32_t hot = left ? 2 * node + 1 : 2 * node + 2;
    int32_t cold = hot == 2 * node + 1 ? 2 * node + 2 : 2 * node + 1;
    double cn = (double)mdl->cover[tb + node];
    double hf = cn > 0 ? (double)mdl->cover[tb + hot] / cn : 0;
    double cf = cn > 0 ? (double)mdl->cover[tb + cold] / cn : 0;
    double iz = 1.0, io = 1.0;
    for (int k = 0; k < len; ++k) {
        if (m[k].fi == f) { iz = m[k].z; io = m[k].o; len = unwind_path(m, len, k); break; }
    }
    shap_recurse(mdl, tb, hot, m, len, iz * hf, io, f, x, i, rows, data_bins, phi);
    shap_recurse(mdl, tb, cold, m, len, iz * cf, 0.0, f, x, i, rows, data_bins, phi);
}

double orc_shap_bias(const orc_forest *m, float base) {                   /* :56-72 */
    double bias = (double)base;
    int32_t *stack = (int32_t *)malloc(sizeof(int32_t) * (size_t)(m->nodes_per_tree + 2));
    for (int32_t t = 0; t < m->num_trees; ++t) {
        int64_t tb = (int64_t)t * m->nodes_per_tree;
        double total = (double)m->cover[tb];
        if (!(total > 0)) continue;
        double mean = 0;
        int sp = 0;
        stack[sp++] = 0;
        while (sp > 0) {
            int32_t n = stack[--sp];
            if (m->feature[tb + n] >= 0) { stack[sp++] = 2 * n + 1; stack[sp++] = 2 * n + 2; }
            else mean += (double)m->leaf[tb + n] * (double)m->cover[tb + n] / total;
        }
        bias += mean;
    }
    free(stack);
    return bias;
}

void orc_treeshap(const orc_forest *m, float base, int32_t data_bins, const float *x,
                  int64_t rows, int32_t cols, float *out) {             /* :170-209 */
    int32_t width = cols + 1;
    double bias = orc_shap_bias(m, base);
    /* rows in chunks of 512 over the host cores (SHAP.swift:179-183) */
#pragma omp parallel
    {
        double *phi = (double *)malloc(sizeof(double) * (size_t)width);
        pe_t empty[1];
#pragma omp for schedule(dynamic, 512)
        for (int64_t i = 0; i < rows; ++i) {
            for (int32_t j = 0; j < width; ++j) phi[j] = 0;
            for (int32_t t = 0; t < m->num_trees; ++t) {
                int64_t tb = (int64_t)t * m->nodes_per_tree;
                if (m->cover[tb] > 0)
                    shap_recurse(m, tb, 0, empty, 0, 1.0, 1.0, -1, x, i, rows, data_bins, phi);
            }
            for (int32_t f = 0; f < cols; ++f) out[i * width + f] = (float)phi[f];
            out[i * width + cols] = (float)bias;
        }
        free(phi);
    }
}
