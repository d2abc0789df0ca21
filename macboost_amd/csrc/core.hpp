// core.hpp — host-side types of the MI355X MacBoost library: parameters
// (BoosterParams, Booster.swift:18-64), trees (Booster.swift:114-146), the
// device context and the booster model.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include <rocprofiler-sdk-roctx/roctx.h>

#include "mbk.h"

struct mbk_context;

namespace mb {

// The device and stream of a kernel-seam context (seam.cpp).
int context_device(const mbk_context *ctx);
hipStream_t context_stream(const mbk_context *ctx);

// A named range on the ROCm tracer's marker timeline (rocprofv3
// --marker-trace) around one phase of host work; free when no tool listens.
struct Phase {
    explicit Phase(const char *name) { roctxRangePush(name); }
    ~Phase() { roctxRangePop(); }
    Phase(const Phase &) = delete;
    Phase &operator=(const Phase &) = delete;
};

// Errors carry the reference's message text (MacBoostError.description,
// MetalEngine.swift:11-20).
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};
[[noreturn]] inline void invalid(const std::string &m) { throw Error("Invalid input: " + m); }
[[noreturn]] inline void internal(const std::string &m) { throw Error("Internal error: " + m); }

#define MB_HIP(expr)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            ::mb::internal(std::string(#expr) + " failed: " + hipGetErrorString(e_));        \
    } while (0)

enum Objective : int {
    OBJ_L2 = 0, OBJ_LOGISTIC = 1, OBJ_MAE = 2, OBJ_HUBER = 3, OBJ_QUANTILE = 4,
    OBJ_POISSON = 5, OBJ_TWEEDIE = 6, OBJ_MULTICLASS = 7,
};

struct Params {
    int num_trees = 100;
    int max_depth = 6;
    float learning_rate = 0.1f;
    float lambda = 1.0f;
    float min_child_hess = 1.0f;
    float min_split_gain = 0.0f;
    int num_bins = 256;
    int objective = OBJ_L2;
    std::set<int> categorical;
    float cat_smooth = 10.0f;
    bool goss = false;
    float goss_top_rate = 0.2f;
    float goss_other_rate = 0.1f;
    float alpha = 0.9f;
    float tweedie_power = 1.5f;
    float scale_pos_weight = 1.0f;
    float subsample = 1.0f;
    float feature_fraction = 1.0f;
    bool has_monotone = false;
    std::vector<int> monotone;
    std::string metric = "auto";
    int num_classes = 1;
    int num_leaves = 0;              // 0 = level-wise growth
    bool has_allowed = false;
    std::set<int> allowed;
    // C-ABI-only keys (CAPI.swift:20-22, :34)
    int early_stopping_rounds = 0;
    int eval_every = 0;
    bool verbose = false;
    std::string init_model;
};

Params parse_params(const char *json);
void validate_params(const Params &p);     // Booster.swift:262-330
std::string objective_name(int obj);

// A trained tree in implicit-heap layout (Booster.swift:119-146).
struct Tree {
    std::vector<int32_t> feature;
    std::vector<float> threshold;
    std::vector<float> leaf;
    std::vector<uint8_t> flags;
    std::vector<uint32_t> cat_mask;  // 8 words per node, empty without categoricals
    std::vector<float> gain;
    std::vector<float> cover;
};

struct Device {
    int id = 0;
    hipStream_t stream = nullptr;
    hipStream_t copy_stream = nullptr;   // host uploads that overlap work on `stream`
    int num_cus = 0;
    explicit Device(int device_id);
    ~Device();
    Device(const Device &) = delete;
    Device &operator=(const Device &) = delete;
};

// A device with idle streams: one an earlier owner handed back, or a new one
// (the calling thread's current device is set either way).
std::unique_ptr<Device> acquire_device(int device_id);
// Hands a device back for reuse; both its streams must be idle.
void release_device(std::unique_ptr<Device> d);

// Host -> device copy of a pageable buffer on stream s.  Copies of 4 MB or
// more go through pinned staging (host fills overlapping the DMA of the other
// buffer): on return the source has been read and the copy is queued on s
// (work queued on s after it sees the data; other streams must wait for s);
// smaller ones are one hipMemcpyAsync.
void upload(void *dst, const void *src, size_t bytes, hipStream_t s);
// Device -> host copy into a pageable buffer after the work queued on s;
// complete on return (64 MB or more through the pinned staging buffers).
void download(void *dst, const void *src, size_t bytes, hipStream_t s);

// Device memory cache for buffers that are allocated once per fit with the
// same sizes fit after fit (the bin matrices, order entries, partials, ...):
// a released block is kept for the next request of the same byte size on the
// same device instead of going back through hipFree / hipMalloc, which cost
// milliseconds per fit at 10M rows.  The cache holds at most half of the
// device's memory (oldest blocks freed first) and is emptied when a
// hipMalloc fails.  A block must be released only when no queued work uses
// it any more.
void *pool_alloc(size_t bytes, int *device);
void pool_free(void *p, size_t bytes, int device);
void pool_trim();                                     // free every cached block
hipError_t malloc_or_trim(void **p, size_t bytes);    // hipMalloc, once more after pool_trim

template <typename T>
struct DevBuf {
    T *ptr = nullptr;
    size_t n = 0;
    bool pooled = false;     // allocate through the device memory cache
    int device = 0;          // of a pooled block
    DevBuf() = default;
    explicit DevBuf(size_t count) { alloc(count); }
    ~DevBuf() { release(); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : ptr(o.ptr), n(o.n), pooled(o.pooled), device(o.device) {
        o.ptr = nullptr;
        o.n = 0;
    }
    DevBuf &operator=(DevBuf &&o) noexcept {
        if (this != &o) {
            release();
            ptr = o.ptr; n = o.n; pooled = o.pooled; device = o.device;
            o.ptr = nullptr; o.n = 0;
        }
        return *this;
    }
    void alloc(size_t count) {
        release();
        n = count;
        if (!count) return;
        if (pooled) {
            ptr = static_cast<T *>(pool_alloc(count * sizeof(T), &device));
        } else {
            void *p = nullptr;
            MB_HIP(malloc_or_trim(&p, count * sizeof(T)));
            ptr = static_cast<T *>(p);
        }
    }
    void release() {
        if (ptr) {
            if (pooled) pool_free(ptr, n * sizeof(T), device);
            else (void)hipFree(ptr);
        }
        ptr = nullptr;
        n = 0;
    }
    size_t bytes() const { return n * sizeof(T); }
};

// Flattened forest resident on the device (forestBuffers, Booster.swift:1944-1985).
struct ForestCache {
    bool valid = false;
    int nodes_per_tree = 0;
    int num_trees = 0;
    bool has_mask = false;
    DevBuf<int32_t> feature;
    DevBuf<float> threshold;
    DevBuf<uint8_t> flags;
    DevBuf<float> leaf;
    DevBuf<uint32_t> mask;
};

struct Booster {
    Params params;
    std::vector<Tree> trees;
    float base_score = 0.0f;
    int num_features = 0;
    int trained_num_bins = 256;
    std::set<int> trained_categorical;
    std::vector<float> base_scores{0.0f};
    int trained_num_classes = 1;
    bool has_feature_names = false;
    std::vector<std::string> feature_names;
    int best_iteration = -1;         // -1 = nil
    std::vector<float> eval_history;
    std::vector<std::string> warnings;

    std::unique_ptr<Device> dev;
    ForestCache forest;

    Booster() = default;
    Booster(const Booster &) = delete;
    Booster &operator=(const Booster &) = delete;
    ~Booster();
    Device &device();
    void build_forest();
    std::vector<float> predict(const float *x_fm, int64_t rows, int64_t cols);
    std::vector<float> predict_raw(const float *x_fm, int64_t rows, int64_t cols);
    void predict_contrib(const float *x_fm, int64_t rows, int64_t cols, float *out);
    std::vector<float> feature_importance(int type) const;
    double shap_bias(int k = 0) const;
    void contrib_class(const float *x_fm, int64_t rows, int64_t cols, int k, float *out);
    std::string to_json() const;
    static Booster *from_json(const std::string &text);
};

// A preprocessed training set (BinnedDataset, Dataset.swift:11-24): bins in
// the tile-8 layout [ceil(cols/8)][rows][8], edges cols*(num_bins-2), labels.
struct BinnedDataset {
    int64_t rows = 0;
    int64_t cols = 0;
    int32_t num_bins = 256;
    std::vector<int32_t> categorical;        // ascending
    bool has_feature_names = false;
    std::vector<std::string> feature_names;
    std::vector<float> labels;
    std::vector<uint8_t> bins;
    std::vector<float> edges;
};
BinnedDataset *dataset_make(const Params &p, const float *x, int64_t rows, int64_t cols,
                            bool row_major, const float *y,
                            const std::vector<std::string> *feature_names);
void dataset_save(const BinnedDataset &ds, const std::string &path);
BinnedDataset *dataset_load(const std::string &path);

Booster *load_model_file(const std::string &path);

// Root-to-leaf path tables of trees first, first + step, ... for the TreeSHAP
// kernels; max_elems is the longest path's split count.
struct ShapTables {
    std::vector<mbk::ShapPath> paths;
    std::vector<mbk::ShapElem> elems;
    std::vector<mbk::ShapUniq> uniq;
    int32_t max_elems = 1;
};
ShapTables shap_tables(const std::vector<Tree> &trees, size_t first, size_t step,
                       int nodes_per_tree);

// Incremental trainer (fitImpl, Booster.swift:445-1701).
struct Trainer;
Trainer *trainer_create(const Params &p, const float *x, int64_t rows, int64_t cols,
                        bool row_major, const float *y, const float *w, const float *xv,
                        int64_t vrows, const float *yv);
// The same with x in device memory (strided as x): nothing is uploaded.
Trainer *trainer_create_device(const Params &p, const float *x_dev, int64_t rows, int64_t cols,
                               bool row_major, const float *y, const float *w, const float *xv,
                               int64_t vrows, const float *yv);
Trainer *trainer_create_binned(const Params &p, const BinnedDataset &ds, const float *w,
                               const float *xv, int64_t vrows, const float *yv);
Trainer *trainer_create_fm(const Params &p, int64_t rows, int64_t cols, const uint8_t *fm_dev,
                           const std::vector<float> &edges, const float *y, const float *w);

// Boruta feature selection (FeatureSelection.swift:45-190): per feature the
// rounds it beat the best shadow, the decision (2 confirmed, 1 tentative,
// 0 rejected) and the gain ratio against the mean best-shadow gain.
struct SelectionResult {
    std::vector<int32_t> hits, decision;
    std::vector<float> gain_ratio;
};
SelectionResult select_features(const Params &p, const float *x_fm, int64_t rows, int64_t cols,
                                const float *y, const float *w, int rounds, int trees,
                                double alpha, uint64_t seed);
void validate_label_values(const Params &p, const float *y, int64_t n);
void trainer_grow(Trainer *t, int num_trees);
// every > 0: time the histogram launches of every every-th tree from now on.
void trainer_profile(Trainer *t, int every);
void trainer_hist_stats(Trainer *t, int64_t *launches, double *ms, double *bytes);
void trainer_level_stats(Trainer *t, int32_t max_levels, int64_t *built, int64_t *active,
                         double *hist_ms);
void trainer_setup_seconds(Trainer *t, double *edges_s, double *bin_s);
Booster *trainer_booster(Trainer *t);
void trainer_free(Trainer *t);
int trainer_classes(const Trainer *t);    // trees per boosting round

// Shared helpers.
void validate_categoricals(const Params &p, const float *x, int64_t rows, int64_t cols,
                           int64_t rs, int64_t cs);
std::string swift_float(float v);
int host_threads();

}  // namespace mb
