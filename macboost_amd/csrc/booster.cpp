// booster.cpp — parameters, the booster model (predict, TreeSHAP, importance,
// model JSON) and every exported C entry point of libmacboostc.so.
//
// Inference always runs on the MI355X: predict_forest and the TreeSHAP kernel
// reproduce the reference's CPU semantics (predictCPU, Booster.swift:2035-2074;
// recursive TreeSHAP, SHAP.swift:170-325) on the device, so there is no
// host-side compute path to fall back to.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <fstream>
#include <sstream>
#include <thread>

#include "../../include/macboost.h"
#include "abi.hpp"
#include "core.hpp"
#include "json.hpp"

namespace mb {

// ---------------------------------------------------------------------------
// parameters (CAPI.swift:9-75, Booster.swift:262-330)
// ---------------------------------------------------------------------------

std::string objective_name(int obj) {
    switch (obj) {
    case OBJ_L2: return "regression";
    case OBJ_LOGISTIC: return "binaryLogistic";
    case OBJ_MAE: return "mae";
    case OBJ_HUBER: return "huber";
    case OBJ_QUANTILE: return "quantile";
    case OBJ_POISSON: return "poisson";
    case OBJ_TWEEDIE: return "tweedie";
    case OBJ_MULTICLASS: return "multiclass";
    }
    return "unknown";
}

static int json_int(const mbjson::Value &v, const char *key) {
    if (v.kind != mbjson::Value::Number || v.num != std::floor(v.num))
        internal(std::string("parameter '") + key + "' must be an integer");
    return (int)v.num;
}
static float json_float(const mbjson::Value &v, const char *key) {
    if (v.kind != mbjson::Value::Number)
        internal(std::string("parameter '") + key + "' must be a number");
    return mbjson::as_float(v);
}
static bool json_bool(const mbjson::Value &v, const char *key) {
    if (v.kind != mbjson::Value::Bool) internal(std::string("parameter '") + key + "' must be a bool");
    return v.b;
}
static std::vector<int> json_ints(const mbjson::Value &v, const char *key) {
    if (v.kind != mbjson::Value::Array) internal(std::string("parameter '") + key + "' must be an array");
    std::vector<int> out;
    for (const auto &e : v.arr) out.push_back(json_int(e, key));
    return out;
}

Params parse_params(const char *json) {
    Params p;
    if (!json) return p;
    mbjson::Value cfg;
    try {
        cfg = mbjson::parse(json);
    } catch (const std::exception &e) {
        internal(e.what());
    }
    if (cfg.kind != mbjson::Value::Object) internal("parameters must be a JSON object");
    std::string objective = "regression";
    for (const auto &kv : cfg.obj) {
        const std::string &k = kv.first;
        const mbjson::Value &v = kv.second;
        if (v.kind == mbjson::Value::Null) continue;
        if (k == "num_trees") p.num_trees = json_int(v, "num_trees");
        else if (k == "max_depth") p.max_depth = json_int(v, "max_depth");
        else if (k == "learning_rate") p.learning_rate = json_float(v, "learning_rate");
        else if (k == "lambda") p.lambda = json_float(v, "lambda");
        else if (k == "min_child_weight") p.min_child_hess = json_float(v, "min_child_weight");
        else if (k == "min_split_gain") p.min_split_gain = json_float(v, "min_split_gain");
        else if (k == "num_bins") p.num_bins = json_int(v, "num_bins");
        else if (k == "objective") {
            if (v.kind != mbjson::Value::String) internal("parameter 'objective' must be a string");
            objective = v.str;
        } else if (k == "categorical_features") {
            auto c = json_ints(v, "categorical_features");
            p.categorical = std::set<int>(c.begin(), c.end());
        } else if (k == "cat_smooth") p.cat_smooth = json_float(v, "cat_smooth");
        else if (k == "early_stopping_rounds") p.early_stopping_rounds = json_int(v, k.c_str());
        else if (k == "eval_every") p.eval_every = json_int(v, "eval_every");
        else if (k == "verbose") p.verbose = json_bool(v, "verbose");
        else if (k == "goss") p.goss = json_bool(v, "goss");
        else if (k == "goss_top_rate") p.goss_top_rate = json_float(v, "goss_top_rate");
        else if (k == "goss_other_rate") p.goss_other_rate = json_float(v, "goss_other_rate");
        else if (k == "alpha") p.alpha = json_float(v, "alpha");
        else if (k == "tweedie_variance_power") p.tweedie_power = json_float(v, k.c_str());
        else if (k == "scale_pos_weight") p.scale_pos_weight = json_float(v, k.c_str());
        else if (k == "subsample") p.subsample = json_float(v, "subsample");
        else if (k == "feature_fraction") p.feature_fraction = json_float(v, "feature_fraction");
        else if (k == "monotone_constraints") {
            p.monotone = json_ints(v, "monotone_constraints");
            p.has_monotone = true;
        } else if (k == "metric") {
            // unknown metric names are ignored (CAPI.swift:62)
            static const char *known[] = {"auto", "rmse", "mae", "logloss", "auc", "pinball",
                                          "poisson", "tweedie", "multi_logloss"};
            if (v.kind != mbjson::Value::String) internal("parameter 'metric' must be a string");
            for (const char *m : known)
                if (v.str == m) p.metric = v.str;
        } else if (k == "num_class") p.num_classes = json_int(v, "num_class");
        else if (k == "init_model") {
            if (v.kind != mbjson::Value::String) internal("parameter 'init_model' must be a string");
            p.init_model = v.str;
        } else if (k == "allowed_features") {
            auto a = json_ints(v, "allowed_features");
            p.allowed = std::set<int>(a.begin(), a.end());
            p.has_allowed = true;
        } else if (k == "num_leaves") {
            int nl = json_int(v, "num_leaves");
            if (nl > 0) p.num_leaves = nl;
        }
    }
    if (objective == "regression" || objective == "l2" || objective == "mse") p.objective = OBJ_L2;
    else if (objective == "binary") p.objective = OBJ_LOGISTIC;
    else if (objective == "mae" || objective == "l1" || objective == "regression_l1") p.objective = OBJ_MAE;
    else if (objective == "huber") p.objective = OBJ_HUBER;
    else if (objective == "quantile") p.objective = OBJ_QUANTILE;
    else if (objective == "poisson") p.objective = OBJ_POISSON;
    else if (objective == "tweedie") p.objective = OBJ_TWEEDIE;
    else if (objective == "multiclass" || objective == "softmax") p.objective = OBJ_MULTICLASS;
    else internal("unknown objective '" + objective + "'");
    return p;
}

void validate_params(const Params &p) {
    if (!(p.num_bins >= 4 && p.num_bins <= 256))
        invalid("numBins must be in 4...256, got " + std::to_string(p.num_bins));
    if (!(p.max_depth >= 1 && p.max_depth <= 12))
        invalid("maxDepth must be in 1...12, got " + std::to_string(p.max_depth));
    if (!(p.num_trees >= 1)) invalid("numTrees must be >= 1, got " + std::to_string(p.num_trees));
    if (!(std::isfinite(p.learning_rate) && p.learning_rate > 0))
        invalid("learningRate must be positive and finite");
    if (p.goss) {
        if (!(p.goss_top_rate > 0 && p.goss_other_rate > 0 && p.goss_top_rate + p.goss_other_rate <= 1))
            invalid("GOSS rates must be positive with topRate + otherRate <= 1");
        if (!(p.subsample >= 1)) invalid("goss and subsample are mutually exclusive");
    }
    if (p.objective == OBJ_QUANTILE && !(p.alpha > 0 && p.alpha < 1))
        invalid("quantile alpha must be in (0, 1)");
    if (p.objective == OBJ_TWEEDIE && !(p.tweedie_power > 1 && p.tweedie_power < 2))
        invalid("tweedieVariancePower must be in (1, 2)");
    if (!(p.subsample > 0 && p.subsample <= 1)) invalid("subsample must be in (0, 1]");
    if (!(p.feature_fraction > 0 && p.feature_fraction <= 1)) invalid("featureFraction must be in (0, 1]");
    if (!(p.scale_pos_weight > 0)) invalid("scalePosWeight must be positive");
    if (p.has_monotone)
        for (int c : p.monotone)
            if (c < -1 || c > 1) invalid("monotone constraints must be -1, 0 or +1");
    if (p.num_leaves > 0 && !(p.num_leaves >= 2 && p.num_leaves <= (1 << p.max_depth)))
        invalid("numLeaves must be in 2...2^maxDepth (= " + std::to_string(1 << p.max_depth) +
                "), got " + std::to_string(p.num_leaves));
    if (p.metric == "auc" && p.objective != OBJ_LOGISTIC)
        invalid("auc metric requires the binary objective");
    if (p.objective == OBJ_MULTICLASS) {
        if (!(p.num_classes >= 3 && p.num_classes <= 128))
            invalid("multiclass requires numClasses in 3...128 (use binaryLogistic for 2)");
        if (p.goss) invalid("GOSS is not supported with multiclass yet");
    }
}

// ---------------------------------------------------------------------------
// booster
// ---------------------------------------------------------------------------

Device &Booster::device() {
    if (!dev) dev = acquire_device(0);
    return *dev;
}

Booster::~Booster() {
    if (!dev) return;
    (void)hipStreamSynchronize(dev->stream);
    (void)hipStreamSynchronize(dev->copy_stream);
    forest = ForestCache();                          // its buffers before the device goes
    release_device(std::move(dev));
}

void Booster::build_forest() {                    // forestBuffers, Booster.swift:1950-1985
    if (forest.valid) return;
    Device &d = device();
    int nodes = 1;
    bool has_cats = false;
    for (const auto &t : trees) {
        nodes = std::max<int>(nodes, (int)t.feature.size());
        has_cats = has_cats || !t.cat_mask.empty();
    }
    const size_t nt = trees.size(), total = nt * (size_t)nodes;
    std::vector<int32_t> feat(total, -1);
    std::vector<float> thr(total, 0.0f), leaf(total, 0.0f);
    std::vector<uint8_t> flags(total, 0);
    std::vector<uint32_t> mask(has_cats ? total * 8 : 8, 0u);
    for (size_t t = 0; t < nt; ++t) {
        const Tree &tr = trees[t];
        for (size_t n = 0; n < tr.feature.size(); ++n) {
            const size_t k = t * nodes + n;
            feat[k] = tr.feature[n];
            thr[k] = n < tr.threshold.size() ? tr.threshold[n] : 0.0f;
            leaf[k] = n < tr.leaf.size() ? tr.leaf[n] : 0.0f;
            flags[k] = n < tr.flags.size() ? tr.flags[n] : 0;
            if (has_cats && tr.cat_mask.size() >= (n + 1) * 8)
                for (int w = 0; w < 8; ++w) mask[k * 8 + w] = tr.cat_mask[n * 8 + w];
        }
    }
    forest.feature.alloc(total);
    forest.threshold.alloc(total);
    forest.flags.alloc(total);
    forest.leaf.alloc(total);
    forest.mask.alloc(mask.size());
    MB_HIP(hipMemcpyAsync(forest.feature.ptr, feat.data(), total * 4, hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipMemcpyAsync(forest.threshold.ptr, thr.data(), total * 4, hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipMemcpyAsync(forest.flags.ptr, flags.data(), total, hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipMemcpyAsync(forest.leaf.ptr, leaf.data(), total * 4, hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipMemcpyAsync(forest.mask.ptr, mask.data(), mask.size() * 4, hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipStreamSynchronize(d.stream));
    forest.nodes_per_tree = nodes;
    forest.num_trees = (int)nt;
    forest.has_mask = has_cats;
    forest.valid = true;
}

std::vector<float> Booster::predict(const float *x, int64_t rows, int64_t cols) {
    std::vector<float> out = predict_raw(x, rows, cols);
    if (params.objective == OBJ_POISSON || params.objective == OBJ_TWEEDIE)
        for (auto &v : out) v = std::exp(v);     // Booster.swift:1992-1997
    return out;
}

// Raw scores, row-major [rows][K]; tree t adds to class t % K
// (predict_forest, Shaders.swift:1548-1578).
std::vector<float> Booster::predict_raw(const float *x, int64_t rows, int64_t cols) {
    const int K = std::max(1, trained_num_classes);
    std::vector<float> out((size_t)std::max<int64_t>(rows, 0) * (size_t)K, 0.0f);
    for (int64_t i = 0; i < rows; ++i)
        for (int k = 0; k < K; ++k)
            out[(size_t)(i * K + k)] = K > 1 ? base_scores[(size_t)k] : base_score;
    if (rows > 0 && !trees.empty()) {
        Device &d = device();
        build_forest();
        DevBuf<float> xd((size_t)rows * (size_t)cols), od((size_t)rows * (size_t)K);
        upload(xd.ptr, x, xd.bytes(), d.stream);
        for (int k = 0; k < K; ++k) {
            mbk::ForestDev f{forest.feature.ptr, forest.threshold.ptr, forest.flags.ptr,
                             forest.leaf.ptr, forest.has_mask ? forest.mask.ptr : nullptr,
                             forest.num_trees, forest.nodes_per_tree, k, K, K};
            MB_HIP(mbk::launch_predict_forest(d.stream, f, xd.ptr, rows, trained_num_bins - 1,
                                              K > 1 ? base_scores[(size_t)k] : base_score,
                                              od.ptr + k));
        }
        MB_HIP(hipMemcpyAsync(out.data(), od.ptr, od.bytes(), hipMemcpyDeviceToHost, d.stream));
        MB_HIP(hipStreamSynchronize(d.stream));
    }
    return out;
}

Booster *load_model_file(const std::string &path) {    // MacBooster.load, :2144-2162
    std::ifstream f(path, std::ios::binary);
    if (!f) internal("cannot read " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    return Booster::from_json(ss.str());
}

// Expected raw score of class k: its base + cover-weighted leaf means of its
// trees (SHAP.swift:56-72).
double Booster::shap_bias(int k) const {
    const int K = std::max(1, trained_num_classes);
    double bias = K > 1 ? (double)base_scores[(size_t)k] : (double)base_score;
    for (size_t t = (size_t)k; t < trees.size(); t += (size_t)K) {
        const Tree &tree = trees[t];
        double total = tree.cover.empty() ? 0.0 : (double)tree.cover[0];
        if (!(total > 0)) continue;
        double mean = 0;
        std::vector<int> stack{0};
        while (!stack.empty()) {
            int n = stack.back();
            stack.pop_back();
            if (tree.feature[n] >= 0) { stack.push_back(2 * n + 1); stack.push_back(2 * n + 2); }
            else mean += (double)tree.leaf[n] * (double)tree.cover[n] / total;
        }
        bias += mean;
    }
    return bias;
}

// Root-to-leaf path decomposition (extractShapPaths, SHAP.swift:79-114), with
// each path's repeated features merged into unique slots.
// Contributions [rows][K][cols + 1]: class k from its own trees and bias.
void Booster::predict_contrib(const float *x, int64_t rows, int64_t cols, float *out) {
    const int K = std::max(1, trained_num_classes);
    if (K == 1) {
        contrib_class(x, rows, cols, 0, out);
        return;
    }
    const int64_t width = cols + 1;
    std::vector<float> c((size_t)std::max<int64_t>(rows, 0) * (size_t)width);
    for (int k = 0; k < K; ++k) {
        contrib_class(x, rows, cols, k, c.data());
        for (int64_t i = 0; i < rows; ++i)
            std::memcpy(out + (size_t)((i * K + k) * width), &c[(size_t)(i * width)],
                        (size_t)width * sizeof(float));
    }
}

// TreeSHAP path tables (extractShapPaths, SHAP.swift:79-114) of trees
// first, first + step, ...: one path per reachable leaf, taken leaf by leaf in
// heap order.  A leaf's splits are found by climbing parent links
// ((n - 1) / 2) to the root and stored root first; each element carries the
// cover fraction of the child the path takes (0x100 in its flags when that
// child is the left one), and repeated features on a path share one unique
// slot whose zero fraction is the product of theirs.  A tree whose root is a
// leaf contributes only to the bias.
ShapTables shap_tables(const std::vector<Tree> &trees, size_t first, size_t step,
                       int nodes_per_tree) {
    ShapTables st;
    std::vector<uint8_t> reach;
    std::vector<int> up;
    for (size_t t = first; t < trees.size(); t += step) {
        const Tree &tr = trees[t];
        const int nn = (int)tr.feature.size();
        if (tr.cover.size() != tr.feature.size() || !(tr.cover[0] > 0)) continue;
        reach.assign((size_t)nn, 0);
        reach[0] = 1;
        for (int n = 0; 2 * n + 2 < nn; ++n)
            if (reach[(size_t)n] && tr.feature[(size_t)n] >= 0)
                reach[(size_t)(2 * n + 1)] = reach[(size_t)(2 * n + 2)] = 1;
        for (int leaf = 1; leaf < nn; ++leaf) {
            if (!reach[(size_t)leaf] || tr.feature[(size_t)leaf] >= 0) continue;
            up.clear();
            for (int c = leaf; c > 0; c = (c - 1) / 2) up.push_back(c);
            if (up.size() > 12) internal("TreeSHAP supports paths of at most 12 splits");
            mbk::ShapPath P{};
            P.elem_start = (int32_t)st.elems.size();
            P.num_elem = (int32_t)up.size();
            P.uniq_start = (int32_t)st.uniq.size();
            P.leaf = (double)tr.leaf[(size_t)leaf];
            for (size_t j = up.size(); j-- > 0;) {
                const int child = up[j], parent = (child - 1) / 2;
                const int32_t f = tr.feature[(size_t)parent];
                const double cp = (double)tr.cover[(size_t)parent];
                const double zf = cp > 0 ? (double)tr.cover[(size_t)child] / cp : 0.0;
                int32_t u = 0;
                while (P.uniq_start + u < (int32_t)st.uniq.size() &&
                       st.uniq[(size_t)(P.uniq_start + u)].feature != f)
                    ++u;
                if (P.uniq_start + u == (int32_t)st.uniq.size())
                    st.uniq.push_back(mbk::ShapUniq{f, 0, 1.0});
                st.uniq[(size_t)(P.uniq_start + u)].zero *= zf;
                const uint32_t side = child == 2 * parent + 1 ? 0x100u : 0u;
                st.elems.push_back(mbk::ShapElem{(int32_t)(t * (size_t)nodes_per_tree + (size_t)parent),
                                                 f, tr.threshold[(size_t)parent],
                                                 (uint32_t)tr.flags[(size_t)parent] | side, u, 0});
            }
            P.num_uniq = (int32_t)st.uniq.size() - P.uniq_start;
            st.max_elems = std::max(st.max_elems, P.num_elem);
            st.paths.push_back(P);
        }
    }
    return st;
}

// TreeSHAP of the trees of class k (every tree when K = 1) into out
// [rows][cols + 1].
void Booster::contrib_class(const float *x, int64_t rows, int64_t cols, int k, float *out) {
    const int K = std::max(1, trained_num_classes);
    const int64_t width = cols + 1;
    const float bias = (float)shap_bias(k);
    if (rows <= 0) return;
    build_forest();
    const ShapTables st = shap_tables(trees, (size_t)k, (size_t)K, forest.nodes_per_tree);
    const std::vector<mbk::ShapPath> &paths = st.paths;
    const std::vector<mbk::ShapElem> &elems = st.elems;
    const std::vector<mbk::ShapUniq> &uniq = st.uniq;
    if (paths.empty()) {
        for (int64_t i = 0; i < rows; ++i) {
            std::fill(out + (size_t)(i * width), out + (size_t)(i * width + cols), 0.0f);
            out[(size_t)(i * width + cols)] = bias;
        }
        return;
    }
    Device &d = device();
    DevBuf<float> xd((size_t)rows * (size_t)cols), od((size_t)rows * (size_t)width);
    DevBuf<mbk::ShapPath> pd(paths.size());
    DevBuf<mbk::ShapElem> ed(elems.size());
    DevBuf<mbk::ShapUniq> ud(uniq.size());
    upload(xd.ptr, x, xd.bytes(), d.stream);
    MB_HIP(hipMemcpyAsync(pd.ptr, paths.data(), pd.bytes(), hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipMemcpyAsync(ed.ptr, elems.data(), ed.bytes(), hipMemcpyHostToDevice, d.stream));
    MB_HIP(hipMemcpyAsync(ud.ptr, uniq.data(), ud.bytes(), hipMemcpyHostToDevice, d.stream));
    DevBuf<double> phi;
    if (mbk::treeshap_needs_scratch((int)cols))
        phi.alloc((size_t)((rows + 63) / 64) * 64 * (size_t)cols);
    MB_HIP(mbk::launch_treeshap(d.stream, xd.ptr, rows, (int)cols, trained_num_bins - 1,
                                forest.has_mask ? forest.mask.ptr : nullptr, pd.ptr,
                                (int)paths.size(), st.max_elems, ed.ptr, ud.ptr, bias, od.ptr,
                                phi.ptr));
    download(out, od.ptr, od.bytes(), d.stream);
}

std::vector<float> Booster::feature_importance(int type) const {   // Booster.swift:1926-1940
    std::vector<float> imp((size_t)num_features, 0.0f);
    for (const auto &tree : trees) {
        std::vector<int> stack{0};
        while (!stack.empty()) {
            int n = stack.back();
            stack.pop_back();
            if (tree.feature[n] < 0) continue;
            const int f = tree.feature[n];
            if (f < num_features)
                imp[(size_t)f] += type == 1 ? 1.0f : ((size_t)n < tree.gain.size() ? tree.gain[n] : 0.0f);
            stack.push_back(2 * n + 1);
            stack.push_back(2 * n + 2);
        }
    }
    return imp;
}

// Model file (ModelFile, Booster.swift:2119-2162).
std::string Booster::to_json() const {
    std::string o;
    auto farr = [&](const std::vector<float> &v) {
        o.push_back('[');
        for (size_t i = 0; i < v.size(); ++i) { if (i) o.push_back(','); mbjson::put_float(o, v[i]); }
        o.push_back(']');
    };
    auto iarr = [&](const auto &v) {
        o.push_back('[');
        for (size_t i = 0; i < v.size(); ++i) { if (i) o.push_back(','); o += std::to_string((long long)v[i]); }
        o.push_back(']');
    };
    o += "{\"version\":1,\"objective\":" + std::to_string(params.objective);
    o += ",\"numBins\":" + std::to_string(trained_num_bins);
    o += ",\"baseScore\":";
    mbjson::put_float(o, base_score);
    o += ",\"numFeatures\":" + std::to_string(num_features);
    o += ",\"categorical\":";
    iarr(std::vector<int>(trained_categorical.begin(), trained_categorical.end()));
    if (has_feature_names) {
        o += ",\"featureNames\":[";
        for (size_t i = 0; i < feature_names.size(); ++i) {
            if (i) o.push_back(',');
            mbjson::put_string(o, feature_names[i]);
        }
        o += "]";
    }
    o += ",\"trees\":[";
    for (size_t t = 0; t < trees.size(); ++t) {
        const Tree &tr = trees[t];
        if (t) o.push_back(',');
        o += "{\"feature\":"; iarr(tr.feature);
        o += ",\"threshold\":"; farr(tr.threshold);
        o += ",\"leaf\":"; farr(tr.leaf);
        o += ",\"flags\":"; iarr(tr.flags);
        o += ",\"catMask\":"; iarr(tr.cat_mask);
        o += ",\"gain\":"; farr(tr.gain);
        o += ",\"cover\":"; farr(tr.cover);
        o += "}";
    }
    o += "],\"numClasses\":" + std::to_string(trained_num_classes);
    o += ",\"baseScores\":"; farr(base_scores);
    o += "}";
    return o;
}

Booster *Booster::from_json(const std::string &text) {
    mbjson::Value m;
    try {
        m = mbjson::parse(text);
    } catch (const std::exception &e) {
        internal(std::string("unreadable model file: ") + e.what());
    }
    auto need = [&](const mbjson::Value &obj, const char *k) -> const mbjson::Value & {
        const mbjson::Value *v = obj.get(k);
        if (!v) internal(std::string("model file is missing '") + k + "'");
        return *v;
    };
    const int version = json_int(need(m, "version"), "version");
    const int obj = json_int(need(m, "objective"), "objective");
    if (version != 1 || obj < 0 || obj > 7) internal("unsupported model file");
    auto b = std::make_unique<Booster>();
    Params p;
    p.num_bins = json_int(need(m, "numBins"), "numBins");
    p.objective = obj;
    const mbjson::Value *nc = m.get("numClasses");
    const int num_classes = nc && nc->kind == mbjson::Value::Number ? json_int(*nc, "numClasses") : 1;
    p.num_classes = std::max(num_classes, obj == OBJ_MULTICLASS ? 3 : 1);
    for (int c : json_ints(need(m, "categorical"), "categorical")) p.categorical.insert(c);
    validate_params(p);
    b->params = p;
    b->trained_num_bins = p.num_bins;
    b->trained_categorical = p.categorical;
    b->base_score = json_float(need(m, "baseScore"), "baseScore");
    b->num_features = json_int(need(m, "numFeatures"), "numFeatures");
    if (const mbjson::Value *fn = m.get("featureNames"); fn && fn->kind == mbjson::Value::Array) {
        b->has_feature_names = true;
        for (const auto &s : fn->arr) b->feature_names.push_back(s.str);
    }
    b->trained_num_classes = num_classes;
    if (const mbjson::Value *bs = m.get("baseScores"); bs && bs->kind == mbjson::Value::Array) {
        b->base_scores.clear();
        for (const auto &v : bs->arr) b->base_scores.push_back(json_float(v, "baseScores"));
    } else {
        b->base_scores = {b->base_score};
    }
    const mbjson::Value &trees = need(m, "trees");
    if (trees.kind != mbjson::Value::Array) internal("model 'trees' must be an array");
    for (const auto &tv : trees.arr) {
        Tree tr;
        for (const auto &v : need(tv, "feature").arr) tr.feature.push_back(json_int(v, "feature"));
        for (const auto &v : need(tv, "threshold").arr) tr.threshold.push_back(json_float(v, "threshold"));
        for (const auto &v : need(tv, "leaf").arr) tr.leaf.push_back(json_float(v, "leaf"));
        for (const auto &v : need(tv, "flags").arr) tr.flags.push_back((uint8_t)json_int(v, "flags"));
        for (const auto &v : need(tv, "catMask").arr) tr.cat_mask.push_back((uint32_t)v.num);
        if (const mbjson::Value *g = tv.get("gain"))
            for (const auto &v : g->arr) tr.gain.push_back(json_float(v, "gain"));
        if (const mbjson::Value *c = tv.get("cover"))
            for (const auto &v : c->arr) tr.cover.push_back(json_float(v, "cover"));
        if (tr.feature.empty() || tr.threshold.size() != tr.feature.size() ||
            tr.leaf.size() != tr.feature.size() || tr.flags.size() != tr.feature.size())
            internal("model tree arrays have inconsistent lengths");
        for (size_t n = 0; n < tr.feature.size(); ++n) {
            if (tr.feature[n] < 0) continue;
            if (2 * n + 2 >= tr.feature.size() || tr.feature[n] >= b->num_features)
                internal("model tree has a split without children or with an unknown feature");
            if ((tr.flags[n] & mbk::FLAG_CATEGORICAL) && tr.cat_mask.size() < (n + 1) * 8)
                internal("model tree has a categorical split without a category mask");
        }
        b->trees.push_back(std::move(tr));
    }
    return b.release();
}

}  // namespace mb

// ===========================================================================
// exported C ABI
// ===========================================================================

using mb::Booster;
using mb::guarded;
using mb::set_err;

namespace {
// Process-wide histogram instrumentation of macboost_train (mbx_profile_global):
// every k-th tree of each later fit times its histogram launches with their own
// dispatch timestamps; the totals add up over the fits.
struct GlobalProfile {
    std::mutex m;
    int every = 0;                 // 0: off
    int64_t launches = 0;
    double ms = 0.0, bytes = 0.0;
    int64_t built[16] = {};
    double level_ms[16] = {};
};
GlobalProfile &global_profile() {
    static GlobalProfile g;
    return g;
}
int global_profile_every() {
    GlobalProfile &g = global_profile();
    std::lock_guard<std::mutex> lock(g.m);
    return g.every;
}
void global_profile_add(mb::Trainer *t) {
    int64_t n = 0, built[16];
    double ms = 0, bytes = 0, lms[16];
    mb::trainer_hist_stats(t, &n, &ms, &bytes);
    mb::trainer_level_stats(t, 16, built, nullptr, lms);
    GlobalProfile &g = global_profile();
    std::lock_guard<std::mutex> lock(g.m);
    g.launches += n;
    g.ms += ms;
    g.bytes += bytes;
    for (int d = 0; d < 16; ++d) {
        g.built[d] += built[d];
        g.level_ms[d] += lms[d];
    }
}
}  // namespace


extern "C" {

void *macboost_train(const char *params_json, const float *x, int64_t rows, int64_t cols,
                     int32_t row_major, const float *y, const float *w, const float *x_valid,
                     int64_t valid_rows, const float *y_valid, char **err) {
    return guarded(err, [&]() -> void * {
        if (!x || !y || rows <= 0 || cols <= 0) mb::internal("null or empty training data");
        mb::Params p = mb::parse_params(params_json);
        const int prof = global_profile_every();
        mb::Trainer *t = mb::trainer_create(p, x, rows, cols, row_major != 0, y, w, x_valid,
                                            valid_rows, y_valid);
        try {
            if (prof > 0) mb::trainer_profile(t, prof);
            mb::trainer_grow(t, p.num_trees * mb::trainer_classes(t));
            Booster *b = mb::trainer_booster(t);
            if (prof > 0) global_profile_add(t);
            mb::trainer_free(t);
            return b;
        } catch (...) {
            mb::trainer_free(t);
            throw;
        }
    }, nullptr);
}

// CAPI.swift:138-183.  Returns 0, or 1 with *err set.
int32_t macboost_select_features(const char *params_json, const float *x, int64_t rows,
                                 int64_t cols, const float *y, const float *w, int32_t rounds,
                                 int32_t trees, float alpha, int64_t seed, int32_t *out_hits,
                                 int32_t *out_decision, float *out_gain_ratio, char **err) {
    return guarded(err, [&]() -> int32_t {
        if (!x || !y || rows <= 0 || cols <= 0 || !out_hits || !out_decision || !out_gain_ratio)
            mb::internal("null or empty selection input");
        mb::Params p = mb::parse_params(params_json);
        const mb::SelectionResult r =
            mb::select_features(p, x, rows, cols, y, w, rounds, trees > 0 ? trees : 0,
                                (double)alpha, (uint64_t)seed);
        for (int64_t f = 0; f < cols; ++f) {
            out_hits[f] = r.hits[(size_t)f];
            out_decision[f] = r.decision[(size_t)f];
            out_gain_ratio[f] = r.gain_ratio[(size_t)f];
        }
        return 0;
    }, 1);
}

int32_t macboost_predict(void *handle, const float *x, int64_t rows, int64_t cols, float *out,
                         char **err) {
    if (!handle || !x || !out) { set_err(err, "null argument"); return -1; }
    Booster *b = static_cast<Booster *>(handle);
    if (cols != b->num_features) {
        set_err(err, "model expects " + std::to_string(b->num_features) + " features, got " +
                         std::to_string(cols));
        return -1;
    }
    return guarded(err, [&]() -> int32_t {
        auto p = b->predict(x, rows, cols);
        std::memcpy(out, p.data(), p.size() * sizeof(float));
        return 0;
    }, -1);
}

int64_t macboost_num_classes(void *handle) {
    return handle ? static_cast<Booster *>(handle)->trained_num_classes : -1;
}

int32_t macboost_feature_importance(void *handle, int32_t type, float *out) {
    if (!handle || !out) return -1;
    auto imp = static_cast<Booster *>(handle)->feature_importance(type == 1 ? 1 : 0);
    std::memcpy(out, imp.data(), imp.size() * sizeof(float));
    return 0;
}

int32_t macboost_predict_contrib(void *handle, const float *x, int64_t rows, int64_t cols,
                                 float *out, char **err) {
    if (!handle || !x || !out) { set_err(err, "null argument"); return -1; }
    Booster *b = static_cast<Booster *>(handle);
    if (cols != b->num_features) {
        set_err(err, "model expects " + std::to_string(b->num_features) + " features, got " +
                         std::to_string(cols));
        return -1;
    }
    return guarded(err, [&]() -> int32_t {
        b->predict_contrib(x, rows, cols, out);
        return 0;
    }, -1);
}

int32_t macboost_save(void *handle, const char *path, char **err) {
    if (!handle || !path) { set_err(err, "null argument"); return -1; }
    return guarded(err, [&]() -> int32_t {
        std::string s = static_cast<Booster *>(handle)->to_json();
        std::ofstream f(path, std::ios::binary);
        if (!f) mb::internal(std::string("cannot write ") + path);
        f << s;
        if (!f) mb::internal(std::string("cannot write ") + path);
        return 0;
    }, -1);
}

void *macboost_load(const char *path, char **err) {
    if (!path) { set_err(err, "null path"); return nullptr; }
    return guarded(err, [&]() -> void * { return mb::load_model_file(path); }, nullptr);
}

int64_t macboost_num_trees(void *handle) {
    return handle ? (int64_t) static_cast<Booster *>(handle)->trees.size() : -1;
}
int64_t macboost_num_features(void *handle) {
    return handle ? static_cast<Booster *>(handle)->num_features : -1;
}
int64_t macboost_best_iteration(void *handle) {
    if (!handle) return -1;
    int b = static_cast<Booster *>(handle)->best_iteration;
    return b < 0 ? 0 : b;
}

char *macboost_warnings(void *handle) {
    if (!handle) return nullptr;
    const auto &w = static_cast<Booster *>(handle)->warnings;
    if (w.empty()) return nullptr;
    std::string j;
    for (size_t i = 0; i < w.size(); ++i) { if (i) j += "\n"; j += w[i]; }
    return strdup(j.c_str());
}

void macboost_free(void *handle) { delete static_cast<Booster *>(handle); }
void macboost_free_string(char *s) { free(s); }

// ---------------------------------------------------------------------------
// extensions (the kernel seam mbk_* is in seam.cpp)
// ---------------------------------------------------------------------------

void *mbx_trainer_create(const char *params_json, const float *x, int64_t rows, int64_t cols,
                         int32_t row_major, const float *y, const float *w, const float *x_valid,
                         int64_t valid_rows, const float *y_valid, char **err) {
    return guarded(err, [&]() -> void * {
        if (!x || !y || rows <= 0 || cols <= 0) mb::internal("null or empty training data");
        mb::Params p = mb::parse_params(params_json);
        return mb::trainer_create(p, x, rows, cols, row_major != 0, y, w, x_valid, valid_rows,
                                  y_valid);
    }, nullptr);
}

int mbx_trainer_grow(void *trainer, int32_t num_trees, char **err) {
    if (!trainer) { set_err(err, "null argument"); return -1; }
    return guarded(err, [&]() -> int {
        mb::trainer_grow(static_cast<mb::Trainer *>(trainer), num_trees);
        return 0;
    }, -1);
}

int mbx_profile_global(int32_t enable, char **err) {
    return guarded(err, [&]() -> int {
        GlobalProfile &g = global_profile();
        std::lock_guard<std::mutex> lock(g.m);
        if (enable > 0 && g.every == 0) {
            g.launches = 0;
            g.ms = g.bytes = 0.0;
            for (int d = 0; d < 16; ++d) {
                g.built[d] = 0;
                g.level_ms[d] = 0.0;
            }
        }
        g.every = enable > 0 ? enable : 0;
        return 0;
    }, -1);
}

int mbx_profile_global_stats(int32_t max_levels, int64_t *launches, double *ms, double *bytes,
                             int64_t *built, double *level_ms, char **err) {
    return guarded(err, [&]() -> int {
        GlobalProfile &g = global_profile();
        std::lock_guard<std::mutex> lock(g.m);
        if (launches) *launches = g.launches;
        if (ms) *ms = g.ms;
        if (bytes) *bytes = g.bytes;
        for (int d = 0; d < max_levels; ++d) {
            if (built) built[d] = d < 16 ? g.built[d] : 0;
            if (level_ms) level_ms[d] = d < 16 ? g.level_ms[d] : 0.0;
        }
        return 0;
    }, -1);
}

int mbx_trainer_profile(void *trainer, int32_t enable, char **err) {
    if (!trainer) { set_err(err, "null argument"); return -1; }
    mb::trainer_profile(static_cast<mb::Trainer *>(trainer), enable > 0 ? enable : 0);
    return 0;
}

int mbx_trainer_hist_stats(void *trainer, int64_t *launches, double *ms, double *bytes,
                           char **err) {
    if (!trainer) { set_err(err, "null argument"); return -1; }
    return guarded(err, [&]() -> int {
        mb::trainer_hist_stats(static_cast<mb::Trainer *>(trainer), launches, ms, bytes);
        return 0;
    }, -1);
}

int mbx_trainer_level_stats(void *trainer, int32_t max_levels, int64_t *built, int64_t *active,
                            double *hist_ms, char **err) {
    if (!trainer || max_levels < 0) { set_err(err, "null argument"); return -1; }
    return guarded(err, [&]() -> int {
        mb::trainer_level_stats(static_cast<mb::Trainer *>(trainer), max_levels, built, active,
                                hist_ms);
        return 0;
    }, -1);
}

int mbx_trainer_setup_seconds(void *trainer, double *edges_s, double *bin_s) {
    if (!trainer) return -1;
    mb::trainer_setup_seconds(static_cast<mb::Trainer *>(trainer), edges_s, bin_s);
    return 0;
}

void *mbx_trainer_booster(void *trainer, char **err) {
    if (!trainer) { set_err(err, "null argument"); return nullptr; }
    return guarded(err, [&]() -> void * {
        return mb::trainer_booster(static_cast<mb::Trainer *>(trainer));
    }, nullptr);
}

void mbx_trainer_free(void *trainer) { mb::trainer_free(static_cast<mb::Trainer *>(trainer)); }

// --- preprocessed datasets (.mbds) -----------------------------------------

void *mbx_dataset_make(const char *params_json, const float *x, int64_t rows, int64_t cols,
                       int32_t row_major, const float *y, const char *feature_names_json,
                       char **err) {
    return guarded(err, [&]() -> void * {
        mb::Params p = mb::parse_params(params_json);
        std::vector<std::string> names;
        if (feature_names_json) {
            mbjson::Value v;
            try {
                v = mbjson::Parser(feature_names_json).parse();
            } catch (const std::exception &) {
                mb::invalid("featureNames must be a JSON array of strings");
            }
            if (v.kind != mbjson::Value::Array)
                mb::invalid("featureNames must be a JSON array of strings");
            for (const auto &e : v.arr) {
                if (e.kind != mbjson::Value::String)
                    mb::invalid("featureNames must be a JSON array of strings");
                names.push_back(e.str);
            }
        }
        return mb::dataset_make(p, x, rows, cols, row_major != 0, y,
                                feature_names_json ? &names : nullptr);
    }, nullptr);
}

int32_t mbx_dataset_save(void *ds, const char *path, char **err) {
    if (!ds || !path) { set_err(err, "null argument"); return -1; }
    return guarded(err, [&]() -> int32_t {
        mb::dataset_save(*static_cast<mb::BinnedDataset *>(ds), path);
        return 0;
    }, -1);
}

void *mbx_dataset_load(const char *path, char **err) {
    if (!path) { set_err(err, "null argument"); return nullptr; }
    return guarded(err, [&]() -> void * { return mb::dataset_load(path); }, nullptr);
}

int32_t mbx_dataset_info(void *ds, int64_t *rows, int64_t *cols, int32_t *num_bins,
                         int32_t *num_categorical) {
    if (!ds) return -1;
    const auto *d = static_cast<const mb::BinnedDataset *>(ds);
    if (rows) *rows = d->rows;
    if (cols) *cols = d->cols;
    if (num_bins) *num_bins = d->num_bins;
    if (num_categorical) *num_categorical = (int32_t)d->categorical.size();
    return 0;
}

int32_t mbx_dataset_copy(void *ds, int32_t *categorical, float *labels, float *edges,
                         uint8_t *bins) {
    if (!ds) return -1;
    const auto *d = static_cast<const mb::BinnedDataset *>(ds);
    if (categorical && !d->categorical.empty())
        std::memcpy(categorical, d->categorical.data(), d->categorical.size() * 4);
    if (labels && !d->labels.empty()) std::memcpy(labels, d->labels.data(), d->labels.size() * 4);
    if (edges && !d->edges.empty()) std::memcpy(edges, d->edges.data(), d->edges.size() * 4);
    if (bins && !d->bins.empty()) std::memcpy(bins, d->bins.data(), d->bins.size());
    return 0;
}

char *mbx_dataset_feature_names(void *ds) {
    if (!ds) return nullptr;
    const auto *d = static_cast<const mb::BinnedDataset *>(ds);
    if (!d->has_feature_names) return nullptr;
    std::string o = "[";
    for (size_t i = 0; i < d->feature_names.size(); ++i) {
        if (i) o += ",";
        mbjson::put_string(o, d->feature_names[i]);
    }
    o += "]";
    return strdup(o.c_str());
}

void *mbx_dataset_train(const char *params_json, void *ds, const float *w, const float *x_valid,
                        int64_t valid_rows, const float *y_valid, char **err) {
    if (!ds) { set_err(err, "null argument"); return nullptr; }
    return guarded(err, [&]() -> void * {
        mb::Params p = mb::parse_params(params_json);
        mb::Trainer *t = mb::trainer_create_binned(p, *static_cast<mb::BinnedDataset *>(ds), w,
                                                   x_valid, valid_rows, y_valid);
        try {
            mb::trainer_grow(t, p.num_trees * mb::trainer_classes(t));
            Booster *b = mb::trainer_booster(t);
            mb::trainer_free(t);
            return b;
        } catch (...) {
            mb::trainer_free(t);
            throw;
        }
    }, nullptr);
}

void mbx_dataset_free(void *ds) { delete static_cast<mb::BinnedDataset *>(ds); }

int64_t mbx_eval_history(void *handle, float *out, int64_t cap) {
    if (!handle) return -1;
    const auto &hist = static_cast<Booster *>(handle)->eval_history;
    const int64_t n = (int64_t)hist.size();
    if (out)
        for (int64_t i = 0; i < std::min(n, cap); ++i) out[i] = hist[(size_t)i];
    return n;
}

void mbx_friedman(int64_t rows, int32_t cols, uint64_t seed, float noise, float *x, float *y) {
    // DataGen.swift:68-94: one SplitMix64 stream per feature, one per
    // 65,536-row noise chunk; every stream is independent, so generate in parallel.
    auto next = [](uint64_t &s) {
        s += 0x9E3779B97F4A7C15ULL;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    };
    auto uni = [&](uint64_t &s) { return (float)(next(s) >> 40) * (1.0f / 16777216.0f); };
    if (cols < 5 || rows <= 0 || !x || !y) return;  // precondition(cols >= 5), DataGen.swift:69
    const int nt = mb::host_threads();
    std::vector<std::thread> th;
    for (int k = 0; k < nt; ++k)
        th.emplace_back([&, k] {
            for (int32_t f = k; f < cols; f += nt) {
                uint64_t s = seed + (uint64_t)f * 0x9E3779B97F4A7C15ULL;
                float *col = x + (int64_t)f * rows;
                for (int64_t i = 0; i < rows; ++i) col[i] = uni(s);
            }
        });
    for (auto &t : th) t.join();
    th.clear();
    const int64_t chunk = 65536, nch = (rows + chunk - 1) / chunk;
    const float pi = 3.14159274101257324f;
    for (int k = 0; k < nt; ++k)
        th.emplace_back([&, k] {
            for (int64_t c = k; c < nch; c += nt) {
                uint64_t s = (seed ^ 0xDEADBEEFULL) + (uint64_t)c * 0x9E3779B97F4A7C15ULL;
                const int64_t end = std::min(rows, (c + 1) * chunk);
                for (int64_t i = c * chunk; i < end; ++i) {
                    float x0 = x[i], x1 = x[rows + i], x2 = x[2 * rows + i];
                    float x3 = x[3 * rows + i], x4 = x[4 * rows + i];
                    float v = 10.0f * sinf(pi * x0 * x1);
                    v = v + 20.0f * (x2 - 0.5f) * (x2 - 0.5f);
                    v = v + 10.0f * x3;
                    v = v + 5.0f * x4;
                    float u1 = uni(s);
                    if (u1 < 1e-7f) u1 = 1e-7f;
                    float u2 = uni(s);
                    y[i] = v + noise * (sqrtf(-2.0f * logf(u1)) * cosf(2.0f * pi * u2));
                }
            }
        });
    for (auto &t : th) t.join();
}

const char *mbx_version(void) { return "macboost-amd 0.1.0 (gfx950)"; }

}  // extern "C"
