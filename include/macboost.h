/*
 * macboost.h — C ABI of the MI355X tree-build library (libmacboostc.so).
 *
 * Part 1 replaces the reference's public C ABI one symbol for one symbol
 * (Sources/MacBoostC/CAPI.swift, MacBoost v1.0.0): same names, argument order,
 * widths, return codes and ownership.  Errors never cross the ABI as
 * exceptions: a failing call stores a malloc'd message in *err (free it with
 * macboost_free_string) and returns NULL / -1 (1 for macboost_select_features).
 * All arrays are borrowed for the duration of the call.  A handle is not safe
 * for concurrent use.
 *
 * Part 2 is the kernel seam (MetalEngine.dispatch, MetalEngine.swift:87-118):
 * device-pointer entry points a host written in another language can drive.
 *
 * Part 3 holds extensions with no counterpart in the reference's C ABI: an
 * incremental trainer used by the benchmark to time boosting iterations with
 * the binned matrix already resident in HBM, and the Swift API's preprocessed
 * datasets (.mbds).
 */
#ifndef MACBOOST_H
#define MACBOOST_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================= Part 1: reference C ABI ======================== */

/* CAPI.swift:86-136.  params_json keys as CAPI.swift:9-37; x is row-major
 * [rows][cols] when row_major != 0 else feature-major [cols][rows]; w,
 * x_valid (feature-major) and y_valid may be NULL.  Returns a handle or NULL. */
void *macboost_train(const char *params_json, const float *x, int64_t rows, int64_t cols,
                     int32_t row_major, const float *y, const float *w, const float *x_valid,
                     int64_t valid_rows, const float *y_valid, char **err);

/* CAPI.swift:138-183 (Boruta feature selection).  Returns 0 / 1. */
int32_t macboost_select_features(const char *params_json, const float *x, int64_t rows,
                                 int64_t cols, const float *y, const float *w, int32_t rounds,
                                 int32_t trees, float alpha, int64_t seed, int32_t *out_hits,
                                 int32_t *out_decision, float *out_gain_ratio, char **err);

/* CAPI.swift:185-202.  x feature-major; out holds rows*num_classes floats. */
int32_t macboost_predict(void *handle, const float *x, int64_t rows, int64_t cols, float *out,
                         char **err);

/* CAPI.swift:204-208.  -1 for a NULL handle. */
int64_t macboost_num_classes(void *handle);

/* CAPI.swift:210-220.  type 0 = gain, 1 = split; out holds num_features. */
int32_t macboost_feature_importance(void *handle, int32_t type, float *out);

/* CAPI.swift:222-240.  out holds rows*num_classes*(cols+1) floats. */
int32_t macboost_predict_contrib(void *handle, const float *x, int64_t rows, int64_t cols,
                                 float *out, char **err);

/* CAPI.swift:242-255 / :257-270: the reference's model JSON. */
int32_t macboost_save(void *handle, const char *path, char **err);
void *macboost_load(const char *path, char **err);

/* CAPI.swift:272-288.  -1 for a NULL handle. */
int64_t macboost_num_trees(void *handle);
int64_t macboost_num_features(void *handle);
int64_t macboost_best_iteration(void *handle);

/* CAPI.swift:290-297: newline-joined fit warnings or NULL; caller frees. */
char *macboost_warnings(void *handle);

/* CAPI.swift:299-308. */
void macboost_free(void *handle);
void macboost_free_string(char *s);

/* ======================= Part 2: kernel seam ============================ */

typedef struct mbk_context mbk_context;

/* One device + one stream.  Replaces MetalEngine.init (MetalEngine.swift:43-65). */
int mbk_context_create(int32_t device, mbk_context **out, char **err);
void mbk_context_destroy(mbk_context *ctx);
int mbk_device_alloc(mbk_context *ctx, size_t bytes, void **out, char **err);
void mbk_device_free(mbk_context *ctx, void *ptr);
int mbk_copy_to_device(mbk_context *ctx, void *dst, const void *src, size_t bytes, char **err);
int mbk_copy_to_host(mbk_context *ctx, void *dst, const void *src, size_t bytes, char **err);
int mbk_synchronize(mbk_context *ctx, char **err);

/* computeEdges (Binner.swift:25-56) on the device: per non-categorical
 * feature, the stride subsample (step = max(1, rows / 200000)) of non-NaN
 * values, sorted; edges[f*(num_bins-2) + k] = sample[min(m-1, (k+1)*m/(num_bins-1))].
 * Categorical and all-NaN features get zero edges.  x is device memory read
 * as x[i*row_stride + f*col_stride]; edges is device memory.  The sort
 * scratch (2 * cols * ceil(rows/step) u32) belongs to the context: it is
 * allocated by the first call that needs more than the context holds. */
int mbk_quantile_edges(mbk_context *ctx, const float *x, int64_t rows, int32_t cols,
                       int64_t row_stride, int64_t col_stride, int32_t num_bins,
                       const uint8_t *is_cat, float *edges, char **err);

/* bin_data (Shaders.swift:46-76): raw f32 -> bins in two layouts, the
 * gather layout bins_tiled [rows][ceil(cols/tile_width)][tile_width] (row-major,
 * each row padded to a whole number of tiles with zero bytes, written by the
 * call) and the
 * feature-major bins_fm [cols][rows].  edges: cols*(num_bins-2) f32. */
int mbk_bin_data(mbk_context *ctx, const float *x, int64_t rows, int32_t cols,
                 int64_t row_stride, int64_t col_stride, const float *edges,
                 const uint8_t *is_cat, int32_t num_bins, int32_t tile_width,
                 uint8_t *bins_tiled, uint8_t *bins_fm, char **err);

/* compute_gradients + quantize_gradients (Shaders.swift:96-192).
 * Writes max_gh[2] (f32 bit patterns of max|g|, max h) and entries[rows][2]
 * = (row, (qg << 16) | qh). */
int mbk_quantize(mbk_context *ctx, int32_t objective, float alpha, float aux,
                 const float *preds, const float *labels, const float *weights, int64_t rows,
                 uint32_t *max_gh, uint32_t *entries, char **err);

/* One split candidate (SplitResult, Shaders.swift:334, plus exact left sums
 * and the categorical left-subset mask). */
typedef struct {
    float gain;
    uint32_t bin;
    float gl, hl;
    uint32_t flags;
    uint32_t pad;
    int64_t gl_int, hl_int;
    uint32_t mask[8];
} mbk_split_result;

/* build_histograms + find_splits for one node (Shaders.swift:212-464): the
 * node's rows are entries[0..n).  hist_out: [num_bins][cols][2] int64
 * (gradient sum, hessian sum) of quantised words; results: [cols].  The
 * histogram scratch belongs to the context, as for mbk_tree_begin. */
int mbk_node_hist_split(mbk_context *ctx, const uint8_t *bins_tiled, int64_t rows,
                        int32_t cols, int32_t num_bins, int32_t tile_width,
                        const uint32_t *entries, int64_t n, const uint32_t *max_gh,
                        const uint8_t *is_cat, const int8_t *monotone, float lambda,
                        float min_child_hess, float cat_smooth, int64_t *hist_out,
                        mbk_split_result *results, char **err);

/* No counterpart in the reference.  mbk_node_hist_split for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same arguments and results,
 * with every scratch buffer in one fixed 16 MiB device array of the library
 * (one per GPU, held until the process ends).  Allocates nothing, fills its
 * scratch with kernels and returns without waiting for the context's stream.
 * Limits: 1..4096 features, and the node's histogram items must fit the
 * array (at tile width 64 and 256 bins: 127 items of 128 KiB, i.e. nodes of
 * up to ~60M rows); larger inputs fail with an error.  Every call on a GPU
 * shares that GPU's array, which keeps the last call's contents: calls that
 * overlap on one GPU (other streams, other threads) race. */
int mbk_node_hist_split_noalloc(mbk_context *ctx, const uint8_t *bins_tiled, int64_t rows,
                                int32_t cols, int32_t num_bins, int32_t tile_width,
                                const uint32_t *entries, int64_t n, const uint32_t *max_gh,
                                const uint8_t *is_cat, const int8_t *monotone, float lambda,
                                float min_child_hess, float cat_smooth, int64_t *hist_out,
                                mbk_split_result *results, char **err);

/* predict_forest (Shaders.swift:1541-1584) on device buffers: flat forest of
 * num_trees*nodes_per_tree heap slots; mask may be NULL when no node is
 * categorical.  x feature-major [cols][rows]; out[rows]. */
int mbk_predict_forest(mbk_context *ctx, const int32_t *feature, const float *threshold,
                       const uint8_t *flags, const float *leaf, const uint32_t *mask,
                       int32_t num_trees, int32_t nodes_per_tree, const float *x, int64_t rows,
                       int32_t data_bins, float base_score, float *out, char **err);

/* ---- one level-wise tree, level by level (fitImpl's level loop,
 * Booster.swift:1467-1648, and the dispatches it encodes, Shaders.swift:
 * 203-464, 1223-1511).  All calls enqueue on the context's stream and return
 * without waiting; split decisions stay on the device.  The caller owns:
 *   bins_tiled  [rows][ceil(cols/tile_width)][tile_width] u8 (mbk_bin_data)
 *   bins_fm     [cols][rows] u8
 *   entries     two buffers of [rows] (row, qg << 16 | qh) u32 pairs; the tree's
 *               rows are the first n_entries of the first (mbk_quantize)
 *   hist        two buffers of [2^(max_depth-1)][num_bins][cols][2] int64
 *   results     [2^(max_depth-1)][cols] mbk_split_result
 *   the tree's model arrays (mbk_tree_out) and preds [rows] f32.
 * The context owns every other buffer (segments, counts, node sums, monotone
 * bounds, partition cursors, histogram items and partials): mbk_tree_begin
 * sizes them when the shape needs more than the context holds, and no other
 * call allocates device memory.  is_cat, monotone and feat_mask are [cols]
 * device arrays or NULL (no categorical, no constraint, every feature).  For
 * level d = 0 .. max_depth-1:
 *   mbk_hist_build(d) -> mbk_hist_subtract(d) -> mbk_find_splits(d) ->
 *   mbk_decide_level(d) -> mbk_route(d)
 * alternating the entries and hist buffers, then mbk_final_leaves.  A call
 * out of this order fails with an error. */
typedef struct {
    int64_t rows;          /* rows of the bin matrices */
    int32_t cols;          /* features */
    int32_t num_bins;      /* bins per feature, the missing bin included: 4..256 */
    int32_t tile_width;    /* features per row tile of bins_tiled: 8, 16, 32 or 64 */
    int32_t max_depth;     /* 1..12 */
} mbk_tree_shape;

typedef struct {           /* BoosterParams (Booster.swift:18-63) */
    float lambda;
    float min_child_hess;
    float min_split_gain;
    float cat_smooth;
    float learning_rate;
} mbk_split_params;

/* NodeSplit (Shaders.swift:466): feature < 0 marks a leaf; flags bit 0 =
 * missing goes left, bit 1 = categorical. */
typedef struct {
    int32_t feature;
    uint32_t bin;
    uint32_t flags;
} mbk_node_split;

/* One tree's model arrays in device memory, heap layout (children of n at
 * 2n+1 and 2n+2, 2^(max_depth+1) - 1 nodes); mask holds 8 words per node. */
typedef struct {
    mbk_node_split *split;
    float *leaf;
    float *gain;
    float *cover;
    uint32_t *mask;
} mbk_tree_out;

/* init_tree (Shaders.swift:1313-1340): level 0 holds the first n_entries
 * entries; max_gh (device, 2 words) are the quantisation maxima. */
int mbk_tree_begin(mbk_context *ctx, const mbk_tree_shape *shape, const uint32_t *max_gh,
                   int64_t n_entries, mbk_tree_out out, char **err);
/* build_histograms (Shaders.swift:203-286): the histograms of level d's
 * built nodes (the smaller child of each split, the root at level 0). */
int mbk_hist_build(mbk_context *ctx, int32_t level, const uint8_t *bins_tiled,
                   const uint32_t *entries, int64_t *hist, char **err);
/* subtract_histograms (Shaders.swift:307-326): each sibling = parent (in
 * hist_prev, the previous level's buffer) - built, exact; nothing at level 0. */
int mbk_hist_subtract(mbk_context *ctx, int32_t level, const int64_t *hist_prev, int64_t *hist,
                      char **err);
/* find_splits + cat_sort (Shaders.swift:328-464): the best split of every
 * (node, feature) of level d. */
int mbk_find_splits(mbk_context *ctx, int32_t level, const int64_t *hist, const uint8_t *is_cat,
                    const int8_t *monotone, const uint8_t *feat_mask,
                    const mbk_split_params *params, mbk_split_result *results, char **err);
/* decide_splits (Shaders.swift:1342-1451): every node of level d splits on
 * its best feature or becomes a leaf; children's sums and monotone bounds. */
int mbk_decide_level(mbk_context *ctx, int32_t level, const mbk_split_result *results,
                     const int8_t *monotone, const mbk_split_params *params, mbk_tree_out out,
                     char **err);
/* route_samples (Shaders.swift:1223-1311): level d's entries partitioned into
 * their children's segments of entries_out, and level d+1 planned (at the
 * last level only the children's rows are counted; entries_out is not
 * written). */
int mbk_route(mbk_context *ctx, int32_t level, const uint8_t *bins_fm, const uint32_t *entries_in,
              uint32_t *entries_out, mbk_tree_out out, char **err);
/* final_leaves (Shaders.swift:1491-1511): leaf values of the deepest level;
 * preds (may be NULL) += the tree, by one walk of every row of bins_fm.
 * Waits for the tree, and fails if a level's histogram items did not fit. */
int mbk_final_leaves(mbk_context *ctx, const uint8_t *bins_fm, const mbk_split_params *params,
                     mbk_tree_out out, float *preds, char **err);
/* The whole tree in one call: mbk_tree_begin, the level loop and
 * mbk_final_leaves.  entries_a holds the tree's entries on entry (it and
 * entries_b are overwritten). */
int mbk_grow_tree(mbk_context *ctx, const mbk_tree_shape *shape, const mbk_split_params *params,
                  const uint8_t *bins_tiled, const uint8_t *bins_fm, const uint8_t *is_cat,
                  const int8_t *monotone, const uint8_t *feat_mask, const uint32_t *max_gh,
                  uint32_t *entries_a, uint32_t *entries_b, int64_t n_entries, int64_t *hist_a,
                  int64_t *hist_b, mbk_split_result *results, mbk_tree_out out, float *preds,
                  char **err);

/* gpuContributions (SHAP.swift:116-166): TreeSHAP of device rows x
 * (feature-major [cols][rows]) under a forest given as host arrays of
 * num_trees*nodes_per_tree heap slots (mask: 8 words per node, NULL without
 * categorical splits); out (device) receives [rows][cols + 1] f32, the bias
 * base_score + the trees' cover-weighted leaf means in the last column.  Path
 * tables and, for more than 4,096 columns, the fp64 accumulators are context
 * scratch. */
int mbk_treeshap(mbk_context *ctx, const int32_t *feature, const float *threshold,
                 const uint8_t *flags, const float *leaf, const float *cover,
                 const uint32_t *mask, int32_t num_trees, int32_t nodes_per_tree,
                 float base_score, int32_t data_bins, const float *x, int64_t rows, int32_t cols,
                 float *out, char **err);

/* fitImpl (Booster.swift:445-1701) over raw features already in device
 * memory: x is read as x[i*cols + f] when row_major != 0, else x[f*rows + i];
 * y, w (nullable) and the feature-major validation set (nullable) are host
 * arrays, as in macboost_train, whose keys, checks and messages apply.  Device
 * quantile edges, binning, every tree and the readback of the model happen
 * inside the call, which first waits for the context's stream.  Returns a
 * booster handle for every Part 1 call (free it with macboost_free), or NULL
 * with *err.  initModel is refused (it needs host features). */
void *mbk_fit(mbk_context *ctx, const char *params_json, const float *x, int64_t rows,
              int64_t cols, int32_t row_major, const float *y, const float *w,
              const float *x_valid, int64_t valid_rows, const float *y_valid, char **err);

/* ======================= Part 3: extensions ============================= */

/* No counterpart in the reference.  An incremental trainer: validates and
 * bins like macboost_train, then grows trees on demand with the binned
 * matrix resident in HBM.  Used to time boosting iterations. */
void *mbx_trainer_create(const char *params_json, const float *x, int64_t rows, int64_t cols,
                         int32_t row_major, const float *y, const float *w,
                         const float *x_valid, int64_t valid_rows, const float *y_valid,
                         char **err);
/* Enqueue num_trees boosting iterations and wait for them. */
int mbx_trainer_grow(void *trainer, int32_t num_trees, char **err);
/* enable = k >= 1: time the histogram launches (their own dispatch
 * timestamps) of every k-th tree from now on; 0: stop. */
int mbx_trainer_profile(void *trainer, int32_t enable, char **err);
/* Histogram-kernel totals over the timed trees since profiling was
 * enabled: launches, total milliseconds, and algorithmic bytes (sum over
 * built nodes of rows*(cols+4)). */
int mbx_trainer_hist_stats(void *trainer, int64_t *launches, double *ms, double *bytes,
                           char **err);
/* Per-level sums over the timed trees since profiling was enabled: rows of
 * built (histogrammed) nodes, live rows, and histogram-kernel milliseconds,
 * levels 0..max_levels-1 (16 at most carry data).  Any output may be NULL. */
int mbx_trainer_level_stats(void *trainer, int32_t max_levels, int64_t *built, int64_t *active,
                            double *hist_ms, char **err);
/* The same instrumentation for fits run with mbk_fit on a context: k >= 1
 * turns it on for every k-th tree (and clears the totals), 0 off.  The
 * totals add up over the fits;
 * built and level_ms (either may be NULL) hold max_levels entries (16 at
 * most carry data): rows of built nodes and histogram milliseconds per level. */
int mbx_context_profile(mbk_context *ctx, int32_t enable, char **err);
int mbx_context_hist_stats(mbk_context *ctx, int32_t max_levels, int64_t *launches, double *ms,
                           double *bytes, int64_t *built, double *level_ms, char **err);
/* The same instrumentation for every macboost_train call of the process
 * from now on: k >= 1 on for every k-th tree of each fit (clearing the
 * totals when it was off), 0 off.  Totals as for mbx_context_hist_stats, added
 * up over the fits since it was turned on.  No counterpart in the reference:
 * it serves timing harnesses that measure the public entry point. */
int mbx_profile_global(int32_t enable, char **err);
int mbx_profile_global_stats(int32_t max_levels, int64_t *launches, double *ms, double *bytes,
                             int64_t *built, double *level_ms, char **err);
/* Wall-clock seconds of the last mbx_trainer_create phases: edges_s the
 * device quantile edges and binning (the label upload overlaps them), bin_s
 * the upload of host features before them (0 for device features). */
int mbx_trainer_setup_seconds(void *trainer, double *edges_s, double *bin_s);
/* Finish training: read the trees back and return a booster handle usable
 * by every Part 1 call (free it with macboost_free).  The trainer stays
 * valid and must still be freed. */
void *mbx_trainer_booster(void *trainer, char **err);
void mbx_trainer_free(void *trainer);

/* Preprocessed datasets: the Swift API's makeDataset / BinnedDataset.save /
 * BinnedDataset.load / fit(dataset:) (Booster.swift:375-436,
 * Dataset.swift:11-86), which the reference's C ABI does not export.
 * mbx_dataset_make validates labels and categoricals, computes quantile edges
 * and bins on the GPU and keeps the bins host-side in the .mbds tile-8 layout
 * [ceil(cols/8)][rows][8]; feature_names_json is a JSON string array or NULL.
 * The file is byte-compatible with the reference's .mbds (little-endian,
 * version 1).  mbx_dataset_train trains with the dataset's bin count,
 * categorical layout and labels (params' num_bins / categorical_features are
 * ignored); w and the feature-major validation set may be NULL.
 * mbx_dataset_copy copies out any non-NULL array: categorical
 * (num_categorical i32, ascending), labels (rows), edges (cols*(num_bins-2)),
 * bins (ceil(cols/8)*rows*8).  mbx_dataset_feature_names returns a JSON array
 * (free with macboost_free_string) or NULL. */
void *mbx_dataset_make(const char *params_json, const float *x, int64_t rows, int64_t cols,
                       int32_t row_major, const float *y, const char *feature_names_json,
                       char **err);
int32_t mbx_dataset_save(void *dataset, const char *path, char **err);
void *mbx_dataset_load(const char *path, char **err);
int32_t mbx_dataset_info(void *dataset, int64_t *rows, int64_t *cols, int32_t *num_bins,
                         int32_t *num_categorical);
int32_t mbx_dataset_copy(void *dataset, int32_t *categorical, float *labels, float *edges,
                         uint8_t *bins);
char *mbx_dataset_feature_names(void *dataset);
void *mbx_dataset_train(const char *params_json, void *dataset, const float *w,
                        const float *x_valid, int64_t valid_rows, const float *y_valid,
                        char **err);
void mbx_dataset_free(void *dataset);

/* The per-iteration validation metric of the fit (MacBooster.evalHistory,
 * Booster.swift:239, :1672): one value per boosting round, including the
 * rounds after the best one that early stopping examined.  Copies at most
 * cap values into out (which may be NULL when cap is 0) and returns the
 * history's length, or -1 for a NULL handle. */
int64_t mbx_eval_history(void *handle, float *out, int64_t cap);

/* SplitMix64 Friedman #1 generator (DataGen.swift:68-94), multithreaded:
 * x feature-major [cols][rows], y[rows]. */
void mbx_friedman(int64_t rows, int32_t cols, uint64_t seed, float noise, float *x, float *y);

/* Library version string (static). */
const char *mbx_version(void);

#ifdef __cplusplus
}
#endif
#endif
