// seam.cpp — the kernel seam (mbk_*): device-pointer entry points a host in
// another language drives, in place of MetalEngine.dispatch
// (MetalEngine.swift:87-118) and the dispatches fitImpl encodes per level
// (Booster.swift:1467-1648).  A context is one device and one stream; it owns
// every scratch buffer the calls need, sized when a call first needs more
// than it holds, so a steady stream of same-shape calls allocates nothing.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

#include "../../include/macboost.h"
#include "abi.hpp"
#include "core.hpp"

using mb::DevBuf;
using mb::guarded;

static_assert(sizeof(mbk_split_result) == sizeof(mbk::SplitResult), "SplitResult layout");
static_assert(sizeof(mbk_node_split) == sizeof(mbk::NodeSplit), "NodeSplit layout");

namespace {

// Grow-only device buffer: reallocated only when a larger size is asked for.
template <typename T>
T *reserve(DevBuf<T> &b, size_t n) {
    if (b.n < n) b.alloc(n);
    return b.ptr;
}

// The level-wise tree in progress and its scratch.
struct TreeScratch {
    DevBuf<mbk::TreeCtl> ctl;
    DevBuf<uint32_t> seg_a, seg_b, count;
    DevBuf<int64_t> node_g, node_h;
    DevBuf<float2> bounds;
    DevBuf<float> cover1;            // the root cover a single-node call does not report
    DevBuf<uint64_t> cursors;
    DevBuf<mbk::Pair> pairs;
    DevBuf<mbk::HistItem> items;
    DevBuf<uint64_t> partials;
    // defaults for NULL is_cat / monotone / feat_mask
    DevBuf<uint8_t> no_cat, all_feats;
    DevBuf<int8_t> no_mono;
    int32_t default_cols = 0;
    // the current tree
    bool active = false;
    mbk::Shape sh{};
    int32_t D = 0;
    int32_t planned = -1;          // level whose built nodes are planned
    int32_t decided = -1;          // last level decided
    uint32_t *seg_cur = nullptr, *seg_next = nullptr;
    uint32_t route_grid = 1, target_items = 1, min_chunk = 2048;
    int hist_grid = 1;
};

struct Scratch {
    TreeScratch tree;
    DevBuf<mbk::TreeCtl> qctl;                       // mbk_quantize
    DevBuf<uint32_t> gmax_part;
    DevBuf<uint32_t> keys_a, keys_b, key_counts;     // mbk_quantile_edges
    DevBuf<mbk::ShapPath> paths;                     // mbk_treeshap
    DevBuf<mbk::ShapElem> elems;
    DevBuf<mbk::ShapUniq> uniq;
    DevBuf<uint32_t> shap_mask;
    DevBuf<double> phi;
};

}  // namespace

struct mbk_context {
    std::unique_ptr<mb::Device> dev;
    Scratch scratch;
    // histogram-kernel timing of the fits run through this context
    bool profiling = false;
    int prof_every = 1;           // profiled fits time every prof_every-th tree
    int64_t prof_launches = 0;
    double prof_ms = 0, prof_bytes = 0;
    int64_t prof_built[16] = {};
    double prof_level_ms[16] = {};
};

namespace {

void need(bool ok, const char *what) {
    if (!ok) mb::invalid(what);
}

mbk::TreeOut tree_out(const mbk_tree_out &o) {
    return mbk::TreeOut{reinterpret_cast<mbk::NodeSplit *>(o.split), o.leaf, o.gain, o.cover,
                        o.mask};
}

mbk::SplitParams split_params(const mbk_split_params *p, int32_t depth) {
    need(p != nullptr, "null split parameters");
    return mbk::SplitParams{p->lambda, p->min_child_hess, p->min_split_gain, p->cat_smooth,
                            p->learning_rate, depth};
}

// The arrays that stand in for NULL is_cat / monotone / feat_mask: no
// categorical feature, no constraint, every feature allowed.
void ensure_defaults(mbk_context *ctx, int32_t cols) {
    TreeScratch &t = ctx->scratch.tree;
    if (t.default_cols >= cols) return;
    hipStream_t s = ctx->dev->stream;
    reserve(t.no_cat, (size_t)cols);
    reserve(t.no_mono, (size_t)cols);
    reserve(t.all_feats, (size_t)cols);
    MB_HIP(hipMemsetAsync(t.no_cat.ptr, 0, (size_t)cols, s));
    MB_HIP(hipMemsetAsync(t.no_mono.ptr, 0, (size_t)cols, s));
    MB_HIP(hipMemsetAsync(t.all_feats.ptr, 1, (size_t)cols, s));
    t.default_cols = cols;
}

// Sizes the tree scratch for `shape` (grow-only) and fills in the tree's
// launch constants; the same decomposition as the trainer's.
void reserve_tree(mbk_context *ctx, const mbk_tree_shape &shape) {
    TreeScratch &t = ctx->scratch.tree;
    const int64_t rows = shape.rows;
    const int32_t cols = shape.cols, nb = shape.num_bins, W = shape.tile_width, D = shape.max_depth;
    mbk::Shape sh{rows, cols, nb, W, (cols + W - 1) / W, 0u, 0, 0, 0};
    mbk::set_hist_tiling(sh);
    const int32_t T = sh.hist_tiles;                 // histogram items per row chunk
    const int64_t level_nodes = (int64_t)1 << (D - 1), total_nodes = ((int64_t)1 << (D + 1)) - 1;
    t.hist_grid = ctx->dev->num_cus;                 // one histogram workgroup per CU
    t.target_items = (uint32_t)t.hist_grid;
    t.min_chunk = 2048;
    int64_t items = T * ((rows + mbk::HIST_CHUNK_MAX - 1) / mbk::HIST_CHUNK_MAX) +
                    t.target_items + 1 + T * level_nodes;
    items = std::min<int64_t>(items, T * ((rows + t.min_chunk - 1) / t.min_chunk + level_nodes + 1));
    t.route_grid = (uint32_t)std::min<int64_t>(
        2 * (int64_t)ctx->dev->num_cus, (rows + mbk::PART_ENTRIES - 1) / mbk::PART_ENTRIES + level_nodes);
    reserve(t.ctl, 1);
    reserve(t.seg_a, (size_t)1 << D);
    reserve(t.seg_b, (size_t)1 << D);
    reserve(t.count, (size_t)total_nodes);
    reserve(t.node_g, (size_t)total_nodes);
    reserve(t.node_h, (size_t)total_nodes);
    reserve(t.bounds, (size_t)total_nodes);
    reserve(t.cursors, (size_t)level_nodes * mbk::CURSOR_STRIDE);
    reserve(t.pairs, (size_t)level_nodes);
    reserve(t.items, (size_t)items);
    reserve(t.partials, (size_t)items * (size_t)sh.part_w * (size_t)nb);
    reserve(t.cover1, 1);
    ensure_defaults(ctx, cols);
    sh.item_cap = (uint32_t)items;
    t.sh = sh;
    t.D = D;
}

void check_shape(const mbk_tree_shape *shape) {
    need(shape != nullptr, "null tree shape");
    need(shape->rows >= 1 && shape->rows <= 0xFFFFFFF0LL, "rows must be in 1..2^32-16");
    need(shape->cols >= 1, "cols must be positive");
    need(shape->num_bins >= 4 && shape->num_bins <= 256, "numBins must be in 4...256");
    need(shape->tile_width == 8 || shape->tile_width == 16 || shape->tile_width == 32 ||
             shape->tile_width == 64,
         "tile_width must be 8, 16, 32 or 64");
    need(shape->max_depth >= 1 && shape->max_depth <= 12, "maxDepth must be in 1...12");
}

// The root plan of a tree of `rows` entries over the scratch of t.
mbk::RootPlan root_plan(const TreeScratch &t, uint32_t rows, float *cover) {
    mbk::RootPlan rp{};
    rp.sh = t.sh;
    rp.rows_active = rows;
    rp.target_items = t.target_items;
    rp.min_chunk = t.min_chunk;
    rp.ctl = t.ctl.ptr;
    rp.seg_start = t.seg_cur;
    rp.count = t.count.ptr;
    rp.pairs = t.pairs.ptr;
    rp.items = t.items.ptr;
    rp.cover = cover;
    rp.bounds = t.bounds.ptr;
    rp.lo = -INFINITY;
    rp.hi = INFINITY;
    return rp;
}

TreeScratch &tree_at(mbk_context *ctx, int32_t level, bool planned_level) {
    need(ctx != nullptr, "null kernel-seam context");
    TreeScratch &t = ctx->scratch.tree;
    need(t.active, "no tree in progress (call mbk_tree_begin first)");
    need(level >= 0 && level < t.D, "level out of range");
    if (planned_level) need(t.planned == level, "level called out of order");
    return t;
}

uint32_t level_pairs(int32_t level) { return level == 0 ? 1u : 1u << (level - 1); }

mbk::LevelArgs level_args(int32_t d, bool terminal) {
    return mbk::LevelArgs{d, (uint32_t)((1u << d) - 1), 1u << d, terminal ? 1u : 0u};
}

// The histogram item list of a level must have fit the scratch: the
// planning kernels report an overflow in the control block.
void check_overflow(mbk_context *ctx) {
    mbk::TreeCtl c{};
    MB_HIP(hipMemcpyAsync(&c, ctx->scratch.tree.ctl.ptr, sizeof c, hipMemcpyDeviceToHost,
                          ctx->dev->stream));
    MB_HIP(hipStreamSynchronize(ctx->dev->stream));
    if (c.overflow) mb::internal("histogram item list overflow");
}

}  // namespace

namespace mb {
int context_device(const mbk_context *ctx) { return ctx->dev->id; }
hipStream_t context_stream(const mbk_context *ctx) { return ctx->dev->stream; }
}  // namespace mb

extern "C" {

int mbk_context_create(int32_t device, mbk_context **out, char **err) {
    return guarded(err, [&]() -> int {
        auto c = std::make_unique<mbk_context>();
        c->dev = std::make_unique<mb::Device>(device);
        *out = c.release();
        return 0;
    }, -1);
}

void mbk_context_destroy(mbk_context *ctx) {
    if (ctx && ctx->dev) (void)hipStreamSynchronize(ctx->dev->stream);
    delete ctx;
}

int mbk_device_alloc(mbk_context *ctx, size_t bytes, void **out, char **err) {
    return guarded(err, [&]() -> int {
        MB_HIP(hipSetDevice(ctx->dev->id));
        MB_HIP(hipMalloc(out, bytes ? bytes : 1));
        return 0;
    }, -1);
}

void mbk_device_free(mbk_context *, void *ptr) {
    if (ptr) (void)hipFree(ptr);
}

int mbk_copy_to_device(mbk_context *ctx, void *dst, const void *src, size_t bytes, char **err) {
    return guarded(err, [&]() -> int {
        MB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->dev->stream));
        MB_HIP(hipStreamSynchronize(ctx->dev->stream));
        return 0;
    }, -1);
}

int mbk_copy_to_host(mbk_context *ctx, void *dst, const void *src, size_t bytes, char **err) {
    return guarded(err, [&]() -> int {
        MB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->dev->stream));
        MB_HIP(hipStreamSynchronize(ctx->dev->stream));
        return 0;
    }, -1);
}

int mbk_synchronize(mbk_context *ctx, char **err) {
    return guarded(err, [&]() -> int {
        MB_HIP(hipStreamSynchronize(ctx->dev->stream));
        return 0;
    }, -1);
}

int mbk_quantile_edges(mbk_context *ctx, const float *x, int64_t rows, int32_t cols,
                       int64_t row_stride, int64_t col_stride, int32_t num_bins,
                       const uint8_t *is_cat, float *edges, char **err) {
    return guarded(err, [&]() -> int {
        if (num_bins < 4 || num_bins > 256) mb::invalid("numBins must be in 4...256");
        if (rows < 1 || cols < 1) mb::invalid("rows and cols must be positive");
        Scratch &sc = ctx->scratch;
        const size_t cap = mbk::edge_sample_cap(rows);
        reserve(sc.keys_a, (size_t)cols * cap);
        reserve(sc.keys_b, (size_t)cols * cap);
        reserve(sc.key_counts, (size_t)cols);
        ensure_defaults(ctx, cols);
        MB_HIP(mbk::launch_edges(ctx->dev->stream, x, rows, cols, row_stride, col_stride,
                                 num_bins, is_cat ? is_cat : sc.tree.no_cat.ptr, sc.keys_a.ptr,
                                 sc.keys_b.ptr, sc.key_counts.ptr, edges));
        MB_HIP(hipStreamSynchronize(ctx->dev->stream));
        return 0;
    }, -1);
}

int mbk_bin_data(mbk_context *ctx, const float *x, int64_t rows, int32_t cols, int64_t row_stride,
                 int64_t col_stride, const float *edges, const uint8_t *is_cat, int32_t num_bins,
                 int32_t tile_width, uint8_t *bins_tiled, uint8_t *bins_fm, char **err) {
    return guarded(err, [&]() -> int {
        if (num_bins < 4 || num_bins > 256) mb::invalid("numBins must be in 4...256");
        const int tiles = (cols + tile_width - 1) / tile_width;
        MB_HIP(mbk::launch_bin_data(ctx->dev->stream, x, rows, cols, row_stride, col_stride, edges,
                                    is_cat, num_bins, tile_width, tiles, bins_tiled, bins_fm));
        return 0;
    }, -1);
}

int mbk_quantize(mbk_context *ctx, int32_t objective, float alpha, float aux, const float *preds,
                 const float *labels, const float *weights, int64_t rows, uint32_t *max_gh,
                 uint32_t *entries, char **err) {
    return guarded(err, [&]() -> int {
        hipStream_t s = ctx->dev->stream;
        if (objective < 0 || objective > 6)
            mb::invalid("mbk_quantize takes objectives 0..6 (one output per row)");
        Scratch &sc = ctx->scratch;
        reserve(sc.qctl, 1);
        reserve(sc.gmax_part, mbk::grad_max_scratch_words());
        mbk::GradParams gp{objective, alpha, aux, weights ? 1 : 0, 1, 0, rows};
        MB_HIP(mbk::launch_tree_init(s, sc.qctl.ptr));
        MB_HIP(mbk::launch_grad_max(s, gp, preds, labels, weights, rows, sc.qctl.ptr,
                                    sc.gmax_part.ptr));
        MB_HIP(mbk::launch_quantize(s, gp, preds, labels, weights, rows, sc.qctl.ptr,
                                    reinterpret_cast<mbk::Entry *>(entries)));
        MB_HIP(hipMemcpyAsync(max_gh, sc.qctl.ptr->max_gh, 8, hipMemcpyDeviceToDevice, s));
        MB_HIP(hipStreamSynchronize(s));
        return 0;
    }, -1);
}

int mbk_tree_begin(mbk_context *ctx, const mbk_tree_shape *shape, const uint32_t *max_gh,
                   int64_t n_entries, mbk_tree_out out, char **err) {
    return guarded(err, [&]() -> int {
        need(ctx != nullptr, "null kernel-seam context");
        check_shape(shape);
        need(n_entries >= 0 && n_entries <= shape->rows, "n_entries must be in 0..rows");
        need(max_gh != nullptr, "null max_gh");
        need(out.split && out.leaf && out.gain && out.cover && out.mask, "null tree array");
        reserve_tree(ctx, *shape);
        TreeScratch &t = ctx->scratch.tree;
        hipStream_t s = ctx->dev->stream;
        const size_t total = ((size_t)1 << (shape->max_depth + 1)) - 1;
        MB_HIP(hipMemsetAsync(out.mask, 0, total * 8 * sizeof(uint32_t), s));
        MB_HIP(mbk::launch_tree_init(s, t.ctl.ptr));
        MB_HIP(hipMemcpyAsync(t.ctl.ptr->max_gh, max_gh, 8, hipMemcpyDeviceToDevice, s));
        t.seg_cur = t.seg_a.ptr;
        t.seg_next = t.seg_b.ptr;
        MB_HIP(mbk::launch_plan_root(s, root_plan(t, (uint32_t)n_entries, out.cover)));
        t.active = true;
        t.planned = 0;
        t.decided = -1;
        return 0;
    }, -1);
}

int mbk_hist_build(mbk_context *ctx, int32_t level, const uint8_t *bins_tiled,
                   const uint32_t *entries, int64_t *hist, char **err) {
    return guarded(err, [&]() -> int {
        TreeScratch &t = tree_at(ctx, level, true);
        hipStream_t s = ctx->dev->stream;
        MB_HIP(mbk::launch_hist(s, t.sh, bins_tiled, reinterpret_cast<const mbk::Entry *>(entries),
                                t.items.ptr, t.ctl.ptr, t.partials.ptr, t.hist_grid));
        MB_HIP(mbk::launch_reduce(s, t.sh, t.pairs.ptr, level_pairs(level), t.partials.ptr,
                                  nullptr, hist, t.ctl.ptr, false));
        return 0;
    }, -1);
}

int mbk_hist_subtract(mbk_context *ctx, int32_t level, const int64_t *hist_prev, int64_t *hist,
                      char **err) {
    return guarded(err, [&]() -> int {
        TreeScratch &t = tree_at(ctx, level, true);
        if (level == 0) return 0;                    // the root has no sibling
        MB_HIP(mbk::launch_subtract(ctx->dev->stream, t.sh, t.pairs.ptr, level_pairs(level),
                                    hist_prev, hist, t.ctl.ptr));
        return 0;
    }, -1);
}

int mbk_find_splits(mbk_context *ctx, int32_t level, const int64_t *hist, const uint8_t *is_cat,
                    const int8_t *monotone, const uint8_t *feat_mask,
                    const mbk_split_params *params, mbk_split_result *results, char **err) {
    return guarded(err, [&]() -> int {
        TreeScratch &t = tree_at(ctx, level, true);
        const mbk::SplitParams sp = split_params(params, t.D);
        MB_HIP(mbk::launch_find_splits(
            ctx->dev->stream, t.sh, sp, t.pairs.ptr, level_pairs(level), hist,
            is_cat ? is_cat : t.no_cat.ptr, monotone ? monotone : t.no_mono.ptr,
            feat_mask ? feat_mask : t.all_feats.ptr, t.ctl.ptr, t.count.ptr, t.node_g.ptr,
            t.node_h.ptr, (1u << level) - 1, reinterpret_cast<mbk::SplitResult *>(results)));
        return 0;
    }, -1);
}

int mbk_decide_level(mbk_context *ctx, int32_t level, const mbk_split_result *results,
                     const int8_t *monotone, const mbk_split_params *params, mbk_tree_out out,
                     char **err) {
    return guarded(err, [&]() -> int {
        TreeScratch &t = tree_at(ctx, level, true);
        const mbk::SplitParams sp = split_params(params, t.D);
        MB_HIP(mbk::launch_decide(ctx->dev->stream, t.sh, sp, level_args(level, false),
                                  reinterpret_cast<const mbk::SplitResult *>(results),
                                  t.count.ptr, t.node_g.ptr, t.node_h.ptr, t.bounds.ptr,
                                  monotone ? monotone : t.no_mono.ptr, t.ctl.ptr,
                                  t.cursors.ptr, tree_out(out)));
        t.decided = level;
        return 0;
    }, -1);
}

int mbk_route(mbk_context *ctx, int32_t level, const uint8_t *bins_fm, const uint32_t *entries_in,
              uint32_t *entries_out, mbk_tree_out out, char **err) {
    return guarded(err, [&]() -> int {
        TreeScratch &t = tree_at(ctx, level, true);
        need(t.decided == level, "mbk_route needs the level's decisions (mbk_decide_level)");
        hipStream_t s = ctx->dev->stream;
        const bool terminal = level + 1 == t.D;
        MB_HIP(mbk::launch_route(s, t.sh, level_args(level, terminal), bins_fm,
                                 reinterpret_cast<const mbk::Entry *>(entries_in),
                                 reinterpret_cast<mbk::Entry *>(entries_out), t.seg_cur,
                                 t.count.ptr, tree_out(out), t.cursors.ptr, t.route_grid,
                                 !terminal));
        MB_HIP(mbk::launch_plan_level(s, t.sh, level_args(level + 1, terminal), t.target_items,
                                      t.min_chunk, t.ctl.ptr, t.seg_cur, t.seg_next, t.count.ptr,
                                      t.cursors.ptr, tree_out(out), t.pairs.ptr, t.items.ptr));
        std::swap(t.seg_cur, t.seg_next);
        t.planned = level + 1;
        return 0;
    }, -1);
}

int mbk_final_leaves(mbk_context *ctx, const uint8_t *bins_fm, const mbk_split_params *params,
                     mbk_tree_out out, float *preds, char **err) {
    return guarded(err, [&]() -> int {
        need(ctx != nullptr, "null kernel-seam context");
        TreeScratch &t = ctx->scratch.tree;
        need(t.active && t.planned == t.D, "mbk_final_leaves needs every level routed");
        hipStream_t s = ctx->dev->stream;
        const mbk::SplitParams sp = split_params(params, t.D);
        const mbk::TreeOut o = tree_out(out);
        MB_HIP(mbk::launch_final_leaves(s, sp, level_args(t.D, true), t.count.ptr, t.node_g.ptr,
                                        t.node_h.ptr, t.bounds.ptr, t.ctl.ptr, o, true));
        if (preds)
            MB_HIP(mbk::launch_predict_binned(s, bins_fm, t.sh.rows, t.sh.num_bins, t.D, o, preds));
        t.active = false;
        check_overflow(ctx);
        return 0;
    }, -1);
}

int mbk_grow_tree(mbk_context *ctx, const mbk_tree_shape *shape, const mbk_split_params *params,
                  const uint8_t *bins_tiled, const uint8_t *bins_fm, const uint8_t *is_cat,
                  const int8_t *monotone, const uint8_t *feat_mask, const uint32_t *max_gh,
                  uint32_t *entries_a, uint32_t *entries_b, int64_t n_entries, int64_t *hist_a,
                  int64_t *hist_b, mbk_split_result *results, mbk_tree_out out, float *preds,
                  char **err) {
    return guarded(err, [&]() -> int {
        char *e = nullptr;
        auto run = [&](int rc) {
            if (rc == 0) return;
            std::string m = e ? e : "Internal error: kernel seam step failed";
            std::free(e);
            throw mb::Error(m);
        };
        run(mbk_tree_begin(ctx, shape, max_gh, n_entries, out, &e));
        uint32_t *ent_cur = entries_a, *ent_next = entries_b;
        int64_t *h_cur = hist_a, *h_prev = hist_b;
        for (int32_t d = 0; d < shape->max_depth; ++d) {
            run(mbk_hist_build(ctx, d, bins_tiled, ent_cur, h_cur, &e));
            run(mbk_hist_subtract(ctx, d, h_prev, h_cur, &e));
            run(mbk_find_splits(ctx, d, h_cur, is_cat, monotone, feat_mask, params, results, &e));
            run(mbk_decide_level(ctx, d, results, monotone, params, out, &e));
            run(mbk_route(ctx, d, bins_fm, ent_cur, ent_next, out, &e));
            std::swap(ent_cur, ent_next);
            std::swap(h_cur, h_prev);
        }
        run(mbk_final_leaves(ctx, bins_fm, params, out, preds, &e));
        return 0;
    }, -1);
}

int mbk_node_hist_split(mbk_context *ctx, const uint8_t *bins_tiled, int64_t rows, int32_t cols,
                        int32_t num_bins, int32_t tile_width, const uint32_t *entries, int64_t n,
                        const uint32_t *max_gh, const uint8_t *is_cat, const int8_t *monotone,
                        float lambda, float min_child_hess, float cat_smooth, int64_t *hist_out,
                        mbk_split_result *results, char **err) {
    return guarded(err, [&]() -> int {
        need(ctx != nullptr, "null kernel-seam context");
        if (n < 0 || n > 0xFFFFFFF0LL) mb::invalid("row count out of range");
        // one node: a depth-1 tree whose root holds entries[0, n)
        const mbk_tree_shape shape{std::max<int64_t>(rows, std::max<int64_t>(n, 1)), cols,
                                   num_bins, tile_width, 1};
        check_shape(&shape);
        reserve_tree(ctx, shape);
        TreeScratch &t = ctx->scratch.tree;
        hipStream_t s = ctx->dev->stream;
        const mbk_split_params sp{lambda, min_child_hess, 0.0f, cat_smooth, 0.1f};
        MB_HIP(mbk::launch_tree_init(s, t.ctl.ptr));
        MB_HIP(hipMemcpyAsync(t.ctl.ptr->max_gh, max_gh, 8, hipMemcpyDeviceToDevice, s));
        t.seg_cur = t.seg_a.ptr;
        t.seg_next = t.seg_b.ptr;
        MB_HIP(mbk::launch_plan_root(s, root_plan(t, (uint32_t)n, t.cover1.ptr)));
        t.active = true;
        t.planned = 0;
        t.decided = -1;
        char *e = nullptr;
        auto run = [&](int rc) {
            if (rc == 0) return;
            std::string m = e ? e : "Internal error: kernel seam step failed";
            std::free(e);
            throw mb::Error(m);
        };
        run(mbk_hist_build(ctx, 0, bins_tiled, entries, hist_out, &e));
        run(mbk_find_splits(ctx, 0, hist_out, is_cat, monotone, nullptr, &sp, results, &e));
        t.active = false;
        check_overflow(ctx);
        return 0;
    }, -1);
}

int mbk_predict_forest(mbk_context *ctx, const int32_t *feature, const float *threshold,
                       const uint8_t *flags, const float *leaf, const uint32_t *mask,
                       int32_t num_trees, int32_t nodes_per_tree, const float *x, int64_t rows,
                       int32_t data_bins, float base_score, float *out, char **err) {
    return guarded(err, [&]() -> int {
        mbk::ForestDev f{feature, threshold, flags, leaf, mask, num_trees, nodes_per_tree, 0, 1, 1};
        MB_HIP(mbk::launch_predict_forest(ctx->dev->stream, f, x, rows, data_bins, base_score, out));
        return 0;
    }, -1);
}

int mbk_treeshap(mbk_context *ctx, const int32_t *feature, const float *threshold,
                 const uint8_t *flags, const float *leaf, const float *cover,
                 const uint32_t *mask, int32_t num_trees, int32_t nodes_per_tree,
                 float base_score, int32_t data_bins, const float *x, int64_t rows, int32_t cols,
                 float *out, char **err) {
    return guarded(err, [&]() -> int {
        need(ctx != nullptr, "null kernel-seam context");
        need(num_trees >= 0 && nodes_per_tree >= 1, "empty forest shape");
        need(rows >= 0 && cols >= 1, "rows and cols must be positive");
        std::vector<mb::Tree> trees((size_t)num_trees);
        const size_t npt = (size_t)nodes_per_tree;
        for (size_t t = 0; t < trees.size(); ++t) {
            mb::Tree &tr = trees[t];
            tr.feature.assign(feature + t * npt, feature + (t + 1) * npt);
            tr.threshold.assign(threshold + t * npt, threshold + (t + 1) * npt);
            tr.flags.assign(flags + t * npt, flags + (t + 1) * npt);
            tr.leaf.assign(leaf + t * npt, leaf + (t + 1) * npt);
            tr.cover.assign(cover + t * npt, cover + (t + 1) * npt);
        }
        // expected raw score: base + each tree's cover-weighted leaf mean
        // (SHAP.swift:56-72)
        double bias = (double)base_score;
        for (const mb::Tree &tr : trees) {
            const double total = (double)tr.cover[0];
            if (!(total > 0)) continue;
            double mean = 0;
            std::vector<int> stack{0};
            while (!stack.empty()) {
                const int n = stack.back();
                stack.pop_back();
                if (tr.feature[(size_t)n] >= 0 && 2 * n + 2 < nodes_per_tree) {
                    stack.push_back(2 * n + 1);
                    stack.push_back(2 * n + 2);
                } else {
                    mean += (double)tr.leaf[(size_t)n] * (double)tr.cover[(size_t)n] / total;
                }
            }
            bias += mean;
        }
        const mb::ShapTables st = mb::shap_tables(trees, 0, 1, nodes_per_tree);
        hipStream_t s = ctx->dev->stream;
        const int64_t width = (int64_t)cols + 1;
        if (rows == 0) return 0;
        Scratch &sc = ctx->scratch;
        if (st.paths.empty()) {
            std::vector<float> row((size_t)width, 0.0f);
            row[(size_t)cols] = (float)bias;
            for (int64_t i = 0; i < rows; ++i)
                MB_HIP(hipMemcpyAsync(out + i * width, row.data(), (size_t)width * 4,
                                      hipMemcpyHostToDevice, s));
            MB_HIP(hipStreamSynchronize(s));
            return 0;
        }
        reserve(sc.paths, st.paths.size());
        reserve(sc.elems, st.elems.size());
        reserve(sc.uniq, st.uniq.size());
        MB_HIP(hipMemcpyAsync(sc.paths.ptr, st.paths.data(), st.paths.size() * sizeof(mbk::ShapPath),
                              hipMemcpyHostToDevice, s));
        MB_HIP(hipMemcpyAsync(sc.elems.ptr, st.elems.data(), st.elems.size() * sizeof(mbk::ShapElem),
                              hipMemcpyHostToDevice, s));
        MB_HIP(hipMemcpyAsync(sc.uniq.ptr, st.uniq.data(), st.uniq.size() * sizeof(mbk::ShapUniq),
                              hipMemcpyHostToDevice, s));
        const uint32_t *mask_dev = nullptr;
        if (mask) {
            const size_t words = (size_t)num_trees * npt * 8;
            reserve(sc.shap_mask, words);
            MB_HIP(hipMemcpyAsync(sc.shap_mask.ptr, mask, words * 4, hipMemcpyHostToDevice, s));
            mask_dev = sc.shap_mask.ptr;
        }
        double *phi = nullptr;
        if (mbk::treeshap_needs_scratch(cols))
            phi = reserve(sc.phi, (size_t)((rows + 63) / 64) * 64 * (size_t)cols);
        MB_HIP(mbk::launch_treeshap(s, x, rows, cols, data_bins, mask_dev, sc.paths.ptr,
                                    (int)st.paths.size(), st.max_elems, sc.elems.ptr, sc.uniq.ptr,
                                    (float)bias, out, phi));
        MB_HIP(hipStreamSynchronize(s));
        return 0;
    }, -1);
}

void *mbk_fit(mbk_context *ctx, const char *params_json, const float *x, int64_t rows,
              int64_t cols, int32_t row_major, const float *y, const float *w,
              const float *x_valid, int64_t valid_rows, const float *y_valid, char **err) {
    return guarded(err, [&]() -> void * {
        need(ctx != nullptr, "null kernel-seam context");
        MB_HIP(hipStreamSynchronize(ctx->dev->stream));
        mb::Params p = mb::parse_params(params_json);
        mb::Trainer *t = mb::trainer_create_device(p, x, rows, cols, row_major != 0, y, w,
                                                   x_valid, valid_rows, y_valid);
        try {
            if (ctx->profiling) mb::trainer_profile(t, ctx->prof_every);
            mb::trainer_grow(t, p.num_trees * mb::trainer_classes(t));
            mb::Booster *b = mb::trainer_booster(t);
            if (ctx->profiling) {
                int64_t n = 0, built[16];
                double ms = 0, bytes = 0, lms[16];
                mb::trainer_hist_stats(t, &n, &ms, &bytes);
                mb::trainer_level_stats(t, 16, built, nullptr, lms);
                ctx->prof_launches += n;
                ctx->prof_ms += ms;
                ctx->prof_bytes += bytes;
                for (int d = 0; d < 16; ++d) {
                    ctx->prof_built[d] += built[d];
                    ctx->prof_level_ms[d] += lms[d];
                }
            }
            mb::trainer_free(t);
            return b;
        } catch (...) {
            mb::trainer_free(t);
            throw;
        }
    }, nullptr);
}

int mbx_context_profile(mbk_context *ctx, int32_t enable, char **err) {
    return guarded(err, [&]() -> int {
        need(ctx != nullptr, "null kernel-seam context");
        if (enable && !ctx->profiling) {
            ctx->prof_launches = 0;
            ctx->prof_ms = ctx->prof_bytes = 0;
            for (int d = 0; d < 16; ++d) {
                ctx->prof_built[d] = 0;
                ctx->prof_level_ms[d] = 0;
            }
        }
        ctx->profiling = enable > 0;
        if (enable > 0) ctx->prof_every = enable;
        return 0;
    }, -1);
}

int mbx_context_hist_stats(mbk_context *ctx, int32_t max_levels, int64_t *launches, double *ms,
                           double *bytes, int64_t *built, double *level_ms, char **err) {
    return guarded(err, [&]() -> int {
        need(ctx != nullptr, "null kernel-seam context");
        if (launches) *launches = ctx->prof_launches;
        if (ms) *ms = ctx->prof_ms;
        if (bytes) *bytes = ctx->prof_bytes;
        for (int d = 0; d < max_levels; ++d) {
            if (built) built[d] = d < 16 ? ctx->prof_built[d] : 0;
            if (level_ms) level_ms[d] = d < 16 ? ctx->prof_level_ms[d] : 0.0;
        }
        return 0;
    }, -1);
}

}  // extern "C"
