/*
 * mbo_oracle.h — CPU restatement of MacBoost's tree-build hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library gives the reference results the HIP
 * implementation in macboost_amd/ is compared with.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * to compare results or as the timed CPU baseline — never as the thing measured
 * or shipped.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the MacBoost v1.0.0 source tree).  Histogram sums are exact integers
 * (int64) over the reference's quantised gradient words, dequantised once per
 * candidate; this is the deterministic summation the HIP path also uses (the
 * reference dequantises per 4096-row group and sums float atomics, which is
 * run-to-run nondeterministic, MacBoostTests.swift:8-10).
 */
#ifndef MBO_ORACLE_H
#define MBO_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_FLAG_DEFAULT_LEFT 1u
#define ORC_FLAG_CATEGORICAL 2u

/* Objectives, numbered as Booster.swift:5-14. */
enum { ORC_OBJ_L2 = 0, ORC_OBJ_LOGISTIC = 1, ORC_OBJ_MAE = 2, ORC_OBJ_HUBER = 3,
       ORC_OBJ_QUANTILE = 4, ORC_OBJ_POISSON = 5, ORC_OBJ_TWEEDIE = 6 };

typedef struct {
    int32_t num_trees;
    int32_t max_depth;
    int32_t num_bins;          /* includes the reserved missing bin */
    int32_t objective;
    int32_t num_leaves;        /* 0 = level-wise growth */
    float learning_rate;
    float lambda;
    float min_child_hess;
    float min_split_gain;
    float cat_smooth;
    float alpha;
    float aux;                 /* scale_pos_weight (logistic) / variance power (tweedie) */
    int32_t goss;              /* 1: GOSS after ceil(1/learning_rate) warm-up trees */
    float goss_top_rate;
    float goss_other_rate;
    float subsample;           /* bagging fraction, 1 = off */
    int32_t num_classes;       /* multiclass K (3..128), else 1 */
    float feature_fraction;    /* per-tree column sample (colsample_bytree), 1 = off */
    int32_t plant;             /* TEST ONLY: a planted mistake (ORC_PLANT_*), 0 = faithful */
    const uint8_t *allowed;    /* [cols] 1 = the feature may split, NULL = every feature */
} orc_params;

/* Planted mistakes, for tests that show a property check catches them.
 * Never set outside tests/. */
#define ORC_PLANT_FIFO_PICK 1      /* leaf-wise: first open leaf with gain > min, not the best */
#define ORC_PLANT_GOSS_NO_SEED 2   /* GOSS/bagging keep hash without the tree seed */
/* quantile edges (orc_compute_edges_planted only) */
#define ORC_PLANT_EDGE_K 3         /* edge k = sample[k*m/dataBins]: one quantile early */
#define ORC_PLANT_EDGE_K2 4        /* edge k = sample[(k+2)*m/dataBins]: one quantile late */
#define ORC_PLANT_EDGE_NUMBINS 5   /* divides by numBins, not numBins - 1 */
#define ORC_PLANT_EDGE_M1 6        /* (k+1)*(m-1)/dataBins: the last index, not the count */
#define ORC_PLANT_EDGE_CEIL 7      /* stride ceil(rows / sampleCap), not the floor */
#define ORC_PLANT_EDGE_NOSTRIDE 8  /* every row sampled */

/* OpenMP threads used by every parallel loop (<= 0: all processors). */
void orc_set_threads(int32_t n);
int32_t orc_get_threads(void);

/* One split candidate result: SplitResult (Shaders.swift:334) plus the exact
 * integer left sums the decision step needs. */
typedef struct {
    float gain;
    uint32_t bin;
    float gl, hl;
    uint32_t flags;
    int64_t gl_int, hl_int;
} orc_split;

/* Flat forest, nodes_per_tree heap slots per tree (Booster.swift:119-146). */
typedef struct {
    int32_t num_trees;
    int32_t nodes_per_tree;
    int32_t *feature;          /* < 0 => leaf */
    float *threshold;
    float *leaf;
    uint8_t *flags;
    uint32_t *cat_mask;        /* 8 words per node, may be NULL */
    float *gain;
    float *cover;
    uint32_t *split_bin;       /* bin of each split (oracle extra, parity aid) */
} orc_forest;

/* --- data generation (DataGen.swift) ------------------------------------ */
uint64_t orc_splitmix_next(uint64_t *state);
float orc_splitmix_uniform(uint64_t *state);
float orc_splitmix_normal(uint64_t *state);
void orc_friedman(int64_t rows, int32_t cols, uint64_t seed, float noise,
                  float *x_fm, float *y);

/* --- binning (Binner.swift, Shaders.swift:46-76) ------------------------- */
void orc_compute_edges(const float *x, int64_t rows, int32_t cols,
                       int64_t row_stride, int64_t col_stride, int32_t num_bins,
                       const uint8_t *is_cat, int64_t sample_cap, float *edges);
/* TEST ONLY: orc_compute_edges with a planted mistake (ORC_PLANT_EDGE_*; 0 = faithful). */
void orc_compute_edges_planted(const float *x, int64_t rows, int32_t cols,
                               int64_t row_stride, int64_t col_stride, int32_t num_bins,
                               const uint8_t *is_cat, int64_t sample_cap, float *edges,
                               int32_t plant);
uint8_t orc_bin_value(float v, const float *edges_f, int32_t num_bins, int is_cat);
void orc_bin_matrix(const float *x, int64_t rows, int32_t cols, int64_t row_stride,
                    int64_t col_stride, const float *edges, const uint8_t *is_cat,
                    int32_t num_bins, uint8_t *bins_fm);

/* --- gradients / quantisation (Shaders.swift:96-192) --------------------- */
float orc_base_score(const float *y, const float *w, int64_t rows, int32_t objective,
                     float scale_pos_weight);
/* L1 / quantile base score: the q-quantile of every max(1, rows/200000)-th
 * label (subsampleQuantile, Booster.swift:786-794). */
float orc_label_quantile(const float *y, int64_t rows, float q);
void orc_gradients(const float *preds, const float *y, const float *w, int64_t rows,
                   int32_t objective, float alpha, float aux, float *g, float *h,
                   float *max_g, float *max_h);
/* Softmax gradients of class c over preds [K][rows] (compute_gradients_multiclass,
 * Shaders.swift:145-170), and the per-class base scores log((1 + w_k) / total)
 * (Booster.swift:841-846). */
void orc_gradients_mc(const float *preds, const float *y, const float *w, int64_t rows,
                      int32_t num_classes, int32_t cls, float *g, float *h, float *max_g,
                      float *max_h);
void orc_base_scores_mc(const float *y, const float *w, int64_t rows, int32_t num_classes,
                        float *out);
void orc_quantize(const float *g, const float *h, int64_t rows, float max_g,
                  float max_h, uint32_t *ghq);

/* --- histogram / split search (Shaders.swift:212-464) ------------------- */
void orc_hist_node(const uint8_t *bins_fm, int64_t rows, int32_t cols, int32_t num_bins,
                   const uint32_t *ghq, const uint32_t *row_idx, int64_t n,
                   int64_t *hg, int64_t *hh);
void orc_find_split(const int64_t *hg, const int64_t *hh, int32_t num_bins, int is_cat,
                    int monotone, int64_t g_tot, int64_t h_tot, float g_inv, float h_inv,
                    float lambda, float min_child_hess, float cat_smooth, orc_split *out);
int32_t orc_cat_order(const int64_t *hg, const int64_t *hh, int32_t num_bins,
                      float g_inv, float h_inv, float cat_smooth, uint16_t *order);

/* --- training (Booster.swift:445-1701 level-wise / :967-1310 leaf-wise) -- */
/* Row sampling for tree `tree` (0-based): goss_grad_hist, goss_threshold and
 * goss_select (Shaders.swift:1093-1221) as driven by Booster.swift:1382-1445.
 * orc_sampling_active says whether the tree samples at all.  g and h are the
 * tree's gradients; amplified rows are scaled in place.  max_g is the
 * unweighted max |g|.  kept[i] = 1 for kept rows; returns their count and the
 * maxima of |g|*w and h*w over them (quantisation uses these). */
int orc_sampling_active(const orc_params *p, int32_t tree);
/* Boruta shadow columns (Shaders.swift:1596-1631): fm [cols][rows] ->
 * fm2 [2*cols][rows], real columns then row-permuted copies. */
uint32_t orc_shadow_perm(uint32_t i, uint32_t n, uint32_t half_bits, uint32_t seed);
void orc_shadow_bins(const uint8_t *fm, int64_t rows, int32_t cols, uint32_t half_bits,
                     uint32_t seed, uint8_t *fm2);
int64_t orc_sample_rows(const orc_params *p, int32_t tree, float *g, float *h, int64_t rows,
                        float max_g, uint8_t *kept, float *wmax_g, float *wmax_h);

/* Multiclass: K trees per round (tree t fits class t % K, its gradients from
 * the preds every earlier tree has updated), preds [K][rows], the forest
 * holds num_trees * K trees. */
int orc_fit(const orc_params *p, const uint8_t *bins_fm, int64_t rows, int32_t cols,
            const float *y, const float *w, const uint8_t *is_cat, const int8_t *monotone,
            const float *edges, float base_score, float *preds, orc_forest *out);

/* --- inference (Booster.swift:2035-2074, SHAP.swift:56-325) ------------ */
void orc_predict(const orc_forest *m, float base_score, int32_t data_bins,
                 const float *x_fm, int64_t rows, int32_t cols, float *out);
void orc_treeshap(const orc_forest *m, float base_score, int32_t data_bins,
                  const float *x_fm, int64_t rows, int32_t cols, float *out);
double orc_shap_bias(const orc_forest *m, float base_score);

#ifdef __cplusplus
}
#endif
#endif
