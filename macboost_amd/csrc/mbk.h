// mbk.h — internal device data structures and kernel launchers of the MI355X
// tree-build path.  Shared by the HIP kernels (kernels_*.hip) and the C++ host
// (booster.cpp).  All structs are plain 4/8-byte-field PODs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mbk {

constexpr uint32_t FLAG_DEFAULT_LEFT = 1u;
constexpr uint32_t FLAG_CATEGORICAL = 2u;

constexpr int PART_ENTRIES = 8192;    // entries per partition block
constexpr int CURSOR_STRIDE = 16;     // u64 words per node cursor (one 128-B line each)
constexpr int SPLIT_KEY_STRIDE = 16;  // u64 words per node split key (one 128-B line each)

// Packed histogram word: (sum of qg) << HIST_QH_BITS + (sum of qh), as a
// 64-bit two's-complement sum.  A histogram item accumulates at most
// HIST_CHUNK_MAX rows, so the hessian field never carries
// (127 * HIST_CHUNK_MAX < 2^27) and the gradient field never overflows
// (32767 * HIST_CHUNK_MAX < 2^36); decode with mask and arithmetic shift.
constexpr int HIST_QH_BITS = 27;
constexpr uint32_t HIST_CHUNK_MAX = (1u << 20) - 1;
static_assert(127ull * HIST_CHUNK_MAX < (1ull << HIST_QH_BITS), "hessian field carries");

// Rows per histogram item for `total` built rows in num_pairs nodes (host
// and device: the planning kernels size a level's items with it, and the
// host can predict the item count).  At most r items per workgroup of the
// grid (target_items): every (pair, tile) adds at most one partial chunk, so
// reserve that slack (T * pairs) and pick the smallest r whose chunk fits
// HIST_CHUNK_MAX.
// The level's item budget, target_items * r: no plan below exceeds it.
__host__ __device__ inline uint64_t item_budget(uint64_t total, uint32_t num_pairs,
                                               int32_t num_tiles, uint32_t target_items) {
    const uint64_t work = total * (uint64_t)num_tiles;
    const uint64_t tgt = target_items ? target_items : 1;
    const uint64_t slack = (uint64_t)num_pairs * (uint64_t)num_tiles;
    const uint64_t need = (work + HIST_CHUNK_MAX - 1) / HIST_CHUNK_MAX;
    uint64_t r = (slack + need + tgt - 1) / tgt;
    if (tgt * r <= slack) r = slack / tgt + 1;
    return tgt * r;
}

__host__ __device__ inline uint32_t item_chunk(uint64_t total, uint32_t num_pairs,
                                               int32_t num_tiles, uint32_t target_items,
                                               uint32_t min_chunk) {
    const uint64_t work = total * (uint64_t)num_tiles;
    const uint64_t slack = (uint64_t)num_pairs * (uint64_t)num_tiles;
    const uint64_t budget = item_budget(total, num_pairs, num_tiles, target_items);
    uint64_t c = (work + (budget - slack) - 1) / (budget - slack);
    if (c < min_chunk) c = min_chunk;
    if (c > HIST_CHUNK_MAX) c = HIST_CHUNK_MAX;
    return (uint32_t)c;
}

// NodeSplit (Shaders.swift:466): feature < 0 marks a leaf.
struct NodeSplit {
    int32_t feature;
    uint32_t bin;
    uint32_t flags;
};

// One (node, feature) split candidate: SplitResult (Shaders.swift:334) plus the
// exact integer left sums and, for categorical splits, the left-subset mask.
struct SplitResult {
    float gain;
    uint32_t bin;
    float gl, hl;
    uint32_t flags;
    uint32_t pad;
    int64_t gl_int, hl_int;
    uint32_t mask[8];
};

// Order entry: a row index travelling with its packed quantised gradient word
// (qg << 16 | qh, Shaders.swift:189-191).
struct Entry {
    uint32_t row;
    uint32_t ghq;
};

// Histogram work item: rows [start, start+count) of the level's order buffer,
// one feature tile, contributing to the built node of `pair`.
struct HistItem {
    uint32_t pair;
    uint32_t tile;
    uint32_t start;
    uint32_t count;
};

// Sibling pair for the split kernel: the built child (histogram from partials),
// the derived child (parent - built) and the parent's slot in the previous
// level's histograms.  derived == 0xFFFFFFFF for the root.
struct Pair {
    uint32_t built;      // level-local node index (slot in hist_cur)
    uint32_t derived;    // level-local node index or NONE
    uint32_t parent;     // slot in hist_prev
    uint32_t item_first; // first HistItem of the built node
    uint32_t nchunks;    // chunks per tile
    uint32_t pad[3];
};
constexpr uint32_t NONE = 0xFFFFFFFFu;

// Global per-fit constants.  The histogram's own tiling (hist_tiles,
// extras, part_w) is derived from the layout's by set_hist_tiling.
struct Shape {
    int64_t rows;        // N
    int32_t cols;        // F
    int32_t num_bins;    // B (incl. missing bin)
    int32_t tile_w;      // W, features per row tile of the gather layout
    int32_t num_tiles;   // T = ceil(F / W)
    uint32_t item_cap;   // capacity of the histogram item list and its partials
    int32_t hist_tiles;  // histogram items per row chunk: T, or T - 1 with extras
    int32_t extras;      // features of the last layout tile folded into the others (0: none)
    int32_t part_w;      // columns of one item's partial: W, or W + 1 / W + 2 with extras
};

// Histogram tiling.  A 32-wide tile costs one ds_add_u64 per 64 rows and
// feature (one row per lane), so the LDS work of a row is its tile count x 32.
// When the last layout tile holds few features (R <= 2 (T - 1), e.g. 4 of 32
// at F = 100), they are not given an item of their own: main tile t also adds
// E_t of them (E_t in {0, 1, 2}; the first max(0, R - (T-1)) tiles take 2),
// which at F = 100 is 34 + 33 + 33 adds per 64 rows instead of 4 x 32.
__host__ __device__ inline int32_t tile_extra_count(const Shape &sh, int32_t t) {
    if (sh.extras == 0) return 0;
    const int32_t e2 = sh.extras > sh.hist_tiles ? sh.extras - sh.hist_tiles : 0;
    return t < e2 ? 2 : (t < sh.extras - e2 ? 1 : 0);
}
// First extra feature of tile t, relative to the last layout tile's first
// feature (hist_tiles * W): tiles with two extras take even offsets.
__host__ __device__ inline int32_t tile_extra_first(const Shape &sh, int32_t t) {
    const int32_t e2 = sh.extras > sh.hist_tiles ? sh.extras - sh.hist_tiles : 0;
    return t + (t < e2 ? t : e2);
}
// The feature that column c of tile t's partial holds, or -1 (padding).
__host__ __device__ inline int32_t partial_feature(const Shape &sh, int32_t t, int32_t c) {
    if (c < sh.tile_w) {
        const int32_t f = t * sh.tile_w + c;
        return f < sh.cols ? f : -1;
    }
    const int32_t e = c - sh.tile_w;
    return e < tile_extra_count(sh, t)
        ? sh.hist_tiles * sh.tile_w + tile_extra_first(sh, t) + e : -1;
}
inline void set_hist_tiling(Shape &sh, bool fold = true) {
    const int32_t last = sh.cols - (sh.num_tiles - 1) * sh.tile_w;   // features of the last tile
    if (fold && sh.tile_w == 32 && sh.num_tiles >= 2 && last <= 2 * (sh.num_tiles - 1)) {
        sh.hist_tiles = sh.num_tiles - 1;
        sh.extras = last;
        sh.part_w = sh.tile_w + (last > sh.hist_tiles ? 2 : 1);
    } else {
        sh.hist_tiles = sh.num_tiles;
        sh.extras = 0;
        sh.part_w = sh.tile_w;
    }
}

struct SplitParams {
    float lambda;
    float min_child_hess;
    float min_split_gain;
    float cat_smooth;
    float learning_rate;
    int32_t max_depth;
};

// Device-resident per-tree control block (counters written by kernels).
struct TreeCtl {
    uint32_t max_gh[2];      // f32 bit patterns of max|g| and max h
    uint32_t num_items;      // histogram items of the current level
    uint32_t num_pairs;      // sibling pairs of the current level
    uint32_t chunk;          // rows per histogram chunk of the current level
    uint32_t overflow;       // 1 when a level needed more items than Shape::item_cap
    uint32_t sampled;        // rows kept by GOSS / bagging for this tree
    uint32_t sample_thr;     // f32 bits of the GOSS keep threshold on |g|
    uint32_t sample_max[2];  // f32 bits of max |g|*w and max h*w over the kept rows
    uint32_t level_active[16];  // live order entries per level
    uint32_t level_built[16];   // rows of built (histogrammed) nodes per level
};

// ---------------------------------------------------------------------------
// Launchers (kernels_*.hip).  All enqueue on `s` and return hipError_t.
// ---------------------------------------------------------------------------

hipError_t launch_bin_data(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                           int64_t row_stride, int64_t col_stride, const float *edges,
                           const uint8_t *is_cat, int32_t num_bins, int32_t tile_w,
                           int32_t num_tiles, uint8_t *bins_tiled, uint8_t *bins_fm);
// Tiles tile_first .. tile_first + tile_count - 1 only (the others untouched).
hipError_t launch_bin_tiles(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                            int64_t rs, int64_t cs, const float *edges, const uint8_t *is_cat,
                            int32_t nb, int32_t tile_w, int32_t num_tiles, int32_t tile_first,
                            int32_t tile_count, uint8_t *tiled, uint8_t *fm);

// Checks of device-resident raw features: a strided row sample
// out[k * cols + f] = x[(k * step) * rs + f * cs] (k < m), and the categorical
// id rule (NaN, or an integer in [0, data_bins)): first_bad[j] (all ones on
// entry) becomes the first row of column cat_cols[j] that breaks it.
hipError_t launch_gather_sample(hipStream_t s, const float *x, int64_t rs, int64_t cs,
                                int64_t step, int64_t m, int32_t cols, float *out);
hipError_t launch_check_categorical(hipStream_t s, const float *x, int64_t rows, int64_t rs,
                                    int64_t cs, const int32_t *cat_cols, int32_t ncat,
                                    int32_t data_bins, uint32_t *first_bad);

// Boruta shadows: fm [cols][rows] -> fm2 [2*cols][rows] (real, then permuted).
hipError_t launch_shadow_bins(hipStream_t s, const uint8_t *fm, int64_t rows, int32_t cols,
                              uint32_t half_bits, uint32_t seed, uint8_t *fm2);

// .mbds tile-8 bins (Dataset.swift:18): feature-major -> [ceil(cols/8)][rows] u64
// words, and back into the gather [rows][T][W] (pre-zeroed) + feature-major
// layouts; *bad (pre-zeroed) becomes nonzero if a bin is >= nb.
hipError_t launch_fm_to_tile8(hipStream_t s, const uint8_t *fm, int64_t rows, int32_t cols,
                              uint64_t *out);
hipError_t launch_tile8_to_layouts(hipStream_t s, const uint64_t *in, int64_t rows, int32_t cols,
                                   int32_t nb, int32_t W, int32_t T, uint8_t *tiled, uint8_t *fm,
                                   uint32_t *bad);

// Quantile edges (Binner.swift:25-56) on the device: x strided as for
// launch_bin_data, edges[cols][num_bins-2] (0 for categorical or all-NaN
// columns).  keys_a / keys_b hold edge_sample_cap(rows) u32 per column (the
// sample keys and the sort's chunk counts); counts (one u32 per column) is
// not used.
size_t edge_sample_cap(int64_t rows);
hipError_t launch_edges(hipStream_t s, const float *x, int64_t rows, int32_t cols, int64_t rs,
                        int64_t cs, int32_t num_bins, const uint8_t *is_cat, uint32_t *keys_a,
                        uint32_t *keys_b, uint32_t *counts, float *edges);

hipError_t launch_tree_init(hipStream_t s, TreeCtl *ctl);
// launch_tree_init in one launch with two neighbours: the previous tree's
// control block first copied to ctl_out (unless null), and with partial the
// gradient maxima reduced as launch_grad_max_final would.
hipError_t launch_tree_start(hipStream_t s, TreeCtl *ctl, TreeCtl *ctl_out,
                             const uint32_t *partial, int nparts);

// Per LABEL block of training rows (k_label_stats): the base score's two
// double sums and the first rejected label / weight row (INT64_MAX: none).
struct LabelStats {
    double s1, s2;
    int64_t bad_label, bad_weight;
};
// label_stats_blocks(rows) entries of out; y, w (nullable) in device memory.
size_t label_stats_blocks(int64_t rows);
hipError_t launch_label_stats(hipStream_t s, int32_t objective, int32_t num_classes,
                              const float *y, const float *w, int64_t rows, float spw,
                              LabelStats *out);

// Objectives numbered as Booster.swift:5-14.
struct GradParams {
    int32_t objective;
    float alpha;
    float aux;
    int32_t has_weights;
    int32_t num_classes;     // multiclass: K, preds are [K][rows]
    int32_t class_index;     // multiclass: the class this tree fits
    int64_t rows;            // multiclass: the class stride of preds
};
// ctl->max_gh = (max |g|, max h); partial: grad_max_scratch_words() u32 of
// device scratch.  With g_out and h_out (rows floats each, 16-B aligned)
// every row's g and h are stored too.
hipError_t launch_grad_max(hipStream_t s, const GradParams &gp, const float *preds,
                           const float *labels, const float *weights, int64_t rows,
                           TreeCtl *ctl, uint32_t *partial, float *g_out = nullptr,
                           float *h_out = nullptr);
size_t grad_max_scratch_words();

// Row sampling (GOSS / bagging) for one tree over the gradients g, h and
// maxima that launch_grad_max stored (g, h 16-B aligned): buckets (1024 u32,
// zero on entry and left zero) hold the |g| histogram; top_count = 0 is
// bagging.  Kept rows
// are compacted into order[0, ctl->sampled), h_kept (rows floats of scratch)
// holds their weighted hessians, ctl->max_gh becomes the weighted maxima over
// kept rows (partial: grad_max_scratch_words() u32), and the entries are
// then quantised in place.  With kept non-null, kept[i] (rows bytes) becomes
// 1 for a kept row and 0 otherwise.
struct SampleParams {
    int32_t goss;            // 1: GOSS histogram threshold; 0: bagging
    uint32_t top_count;      // floor(rows * top_rate) (0 for bagging)
    float other_prob;        // keep probability below the threshold
    float weight;            // amplification of the sampled rest
    uint32_t seed;           // tree index + 1
    uint32_t pad[3];
};
// Per-level view of the heap: level d holds nodes [2^d - 1, 2^(d+1) - 1).
struct LevelArgs {
    int32_t level;           // d
    uint32_t level_start;    // heap index of the level's first node
    uint32_t num_level;      // 2^d
    uint32_t terminal;       // 1: children of the routed level are final leaves
};

struct TreeOut {             // one tree's model arrays (heap layout)
    NodeSplit *split;
    float *leaf;
    float *gain;
    float *cover;
    uint32_t *mask;          // 8 words per node
};

// A finished tree's deepest-level fixup (launch_final_fixup's arguments) left
// to the next tree's root pass; active == 0: none.
struct PendingFixup {
    LevelArgs la;
    const uint32_t *count;
    TreeOut out;
    int32_t zero_empty, active;
};

// The root level's plan (launch_plan_root's arguments): the root node's
// count, segment, cover, bounds, its one pair and its histogram items.
// rows_active == NONE takes ctl->sampled (a sampled tree's kept rows).
struct RootPlan {
    Shape sh;
    uint32_t rows_active, target_items, min_chunk, pad;
    TreeCtl *ctl;
    uint32_t *seg_start, *count;
    Pair *pairs;
    HistItem *items;
    float *cover;
    float2 *bounds;
    float lo, hi;
};
// With plan non-null the last pass (the kept rows' quantiser) also plans the
// root, in its first workgroup; with fix non-null that workgroup first does
// the previous tree's deepest-level fixup.  With walk_part non-null the tree's
// start (launch_tree_start(ctl, ctl_prev, walk_part, walk_nparts)) is left to
// the first pass, which does it itself.
hipError_t launch_sample(hipStream_t s, const SampleParams &sp, int64_t rows, TreeCtl *ctl,
                         uint32_t *buckets, const float *g, const float *h,
                         Entry *order, float *h_kept, uint8_t *kept,
                         const RootPlan *plan = nullptr, const PendingFixup *fix = nullptr,
                         TreeCtl *ctl_prev = nullptr, const uint32_t *walk_part = nullptr,
                         int walk_nparts = 0);
// Every row quantised with ctl->max_gh into order[i] = {i, packed (qg, qh)};
// with implicit_rows, into the u32 words ((uint32_t *)order)[i] = packed
// (qg, qh) only: the root's rows in order, row i being entry i.  With plan
// non-null the first workgroup also plans the root (plan->rows_active rows)
// while the others quantise, after the previous tree's fixup when fix is
// non-null.
hipError_t launch_quantize(hipStream_t s, const GradParams &gp, const float *preds,
                           const float *labels, const float *weights, int64_t rows,
                           const TreeCtl *ctl, Entry *order, bool implicit_rows = false,
                           const RootPlan *plan = nullptr, const PendingFixup *fix = nullptr);

// Where the histogram kernel finds tile t of row r: at
// base + t * tile_step + r * (t == last_tile ? last_stride : stride); with
// extras, the dword holding row r's extra bytes f0..f0+3 (f0 a multiple of 4)
// at base + x_off + r * x_stride + f0.
struct HistLayout {
    int64_t tile_step;
    int32_t stride;
    int32_t last_stride;
    int32_t last_tile;
    int32_t x_stride;
    int64_t x_off;
};
// The gather layout [rows][T][W]: tile_step W, both strides T * W; the
// extras are the last tile's bytes of the row.
HistLayout gather_layout(const Shape &sh);
// The planar root copy (launch_planar_rows).  W = 64, T >= 2: [T][rows][...],
// tile t < T - 1 at t * rows * 64 with stride 64, the last tile with stride
// ceil(F_last/16)*16.  W = 32 with extras: [T-1][rows][32] plus one plane of
// each row's extra bytes, padded to a multiple of 4.  Each tile's bytes are
// then contiguous, so the tile workgroups of a row chunk stream their own
// planes.
bool has_planar_layout(const Shape &sh);
HistLayout planar_layout(const Shape &sh);
size_t planar_bytes(const Shape &sh);    // including 64 zero bytes of overread

// Histogram items -> packed partials [item][B][part_w] (64-bit words, see
// HIST_QH_BITS).  layout null: the gather layout.  With start / stop events
// (created by the caller), they take the kernel's own dispatch timestamps.
// implicit_rows: order holds launch_quantize's implicit u32 words (the root
// of an unsampled tree; entry j is row j).
hipError_t launch_hist(hipStream_t s, const Shape &sh, const uint8_t *bins_tiled,
                       const Entry *order, const HistItem *items, const TreeCtl *ctl,
                       uint64_t *partials, int grid, const HistLayout *layout = nullptr,
                       hipEvent_t start = nullptr, hipEvent_t stop = nullptr,
                       bool implicit_rows = false);
size_t hist_lds_size();   // static LDS of one histogram workgroup (one per CU)
// Planar copy of the gather layout for the root pass over every row; out
// holds planar_bytes(sh) bytes (the last tile's loads run up to 16 B past its
// rows into the zeroed tail, and into the next row's bytes, which land in
// padding columns).
// tiled: rows of row_bytes bytes holding feature f at byte f (the gather
// layout of any tile width: its tiles are contiguous and all but the last full).
hipError_t launch_planar_rows(hipStream_t s, const Shape &sh, const uint8_t *tiled,
                              int32_t row_bytes, uint8_t *out);

// Reduce partials into hist_cur [node][B][F][g,h] (int64), derive siblings
// from hist_prev, then search splits for both nodes of each pair.
// With keys (level-local, node l's at keys[l * SPLIT_KEY_STRIDE]) every node's
// best (gain, feature) is also left there as a split_key maximum, for the next
// partition to decide the level (launch_route with RouteDecide) in place of
// launch_decide; cursors (non-null) are then zeroed for that partition.
hipError_t launch_split(hipStream_t s, const Shape &sh, const SplitParams &sp,
                        const Pair *pairs, uint32_t max_pairs, const uint64_t *partials,
                        const int64_t *hist_prev, int64_t *hist_cur, const uint8_t *is_cat,
                        const int8_t *monotone, const uint8_t *feat_mask,
                        const TreeCtl *ctl, const uint32_t *count, int64_t *node_g,
                        int64_t *node_h, uint32_t level_start, SplitResult *results,
                        uint64_t *keys = nullptr, uint64_t *cursors = nullptr);

// The two halves of launch_split, for the kernel seam: partials -> built
// histograms (and, with derive, the derived siblings), and the split search
// over histograms already in hist_cur; plus the subtraction on its own.
hipError_t launch_reduce(hipStream_t s, const Shape &sh, const Pair *pairs, uint32_t max_pairs,
                         const uint64_t *partials, const int64_t *hist_prev, int64_t *hist_cur,
                         const TreeCtl *ctl, bool derive, uint64_t *keys = nullptr,
                         uint64_t *cursors = nullptr, uint32_t nzero = 0);
hipError_t launch_subtract(hipStream_t s, const Shape &sh, const Pair *pairs, uint32_t max_pairs,
                           const int64_t *hist_prev, int64_t *hist_cur, const TreeCtl *ctl);
hipError_t launch_find_splits(hipStream_t s, const Shape &sh, const SplitParams &sp,
                              const Pair *pairs, uint32_t max_pairs, const int64_t *hist_cur,
                              const uint8_t *is_cat, const int8_t *monotone,
                              const uint8_t *feat_mask, const TreeCtl *ctl, const uint32_t *count,
                              int64_t *node_g, int64_t *node_h, uint32_t level_start,
                              SplitResult *results, uint64_t *keys = nullptr);

hipError_t launch_plan_root(hipStream_t s, const RootPlan &plan);

hipError_t launch_decide(hipStream_t s, const Shape &sh, const SplitParams &sp,
                         const LevelArgs &la, const SplitResult *results,
                         const uint32_t *count, int64_t *node_g, int64_t *node_h,
                         float2 *bounds, const int8_t *monotone, const TreeCtl *ctl,
                         uint64_t *cursors, TreeOut out);

// Deepest level: leaf values of split parents' children, counts zeroed
// (launch_walk_count fills them, launch_final_fixup writes covers).
// counted: the counts come from the partition (sampled trees) instead.
hipError_t launch_final_leaves(hipStream_t s, const SplitParams &sp, const LevelArgs &la,
                               uint32_t *count, const int64_t *node_g,
                               const int64_t *node_h, const float2 *bounds,
                               const TreeCtl *ctl, TreeOut out, bool counted);
// Covers of the level's nodes from count; with zero_empty, empty nodes' leaves
// become 0.
hipError_t launch_final_fixup(hipStream_t s, const LevelArgs &la, const uint32_t *count,
                              TreeOut out, bool zero_empty = true);

// Leaf renewal of the L1 / quantile objectives for one finished tree: the
// sampled rows' residual quantiles replace its leaf values in place.  Scratch:
// leaf_of, keys, seg hold renew_sample_count(rows) u32; cnt, off, cursor
// 2^(max_depth+1)-1 u32.  delta (nodes f32, or null) receives new - old for
// the leaf-wise update of preds that already hold the old leaves.
size_t renew_sample_count(int64_t rows);
hipError_t launch_renew(hipStream_t s, const uint8_t *bins_fm, int64_t rows, int32_t nb,
                        int32_t max_depth, TreeOut tree, const float *labels,
                        const float *preds, const float2 *bounds, float q, float lr,
                        uint32_t *leaf_of, uint32_t *keys, uint32_t *seg, uint32_t *cnt,
                        uint32_t *off, uint32_t *cursor, float *delta);

// Partition of the routed level (d-1): every split node's interval is split
// in place between its children (left from the front, right from the back).
// Node l's cursor is cursors[l * CURSOR_STRIDE]: left count in the low word,
// right count in the high word; the level's k_decide zeroes them.  max_blocks
// is the persistent grid (any size >= 1; each block takes every max_blocks-th
// of the level's PART_ENTRIES-entry blocks).  write_entries = false only
// counts (terminal level).
// With plan, the partition's last workgroup then plans the next level as
// launch_plan_level(plan->next, ...) would, from seg_start into
// plan->seg_next; plan->done is one u32, zero before the launch and zero
// again after it.
struct RoutePlan {
    LevelArgs next;
    uint32_t target_items, min_chunk;
    TreeCtl *ctl;
    uint32_t *seg_next;
    Pair *pairs;
    HistItem *items;
    uint32_t *done;
};
// With decide, the routed level has not been decided yet (launch_split left
// its keys, no launch_decide ran): every workgroup takes each node's split
// from its key and the winning feature's SplitResult, and the nodes' model
// arrays, children's sums and bounds are written here, as launch_decide
// would (the level's cursors were zeroed by launch_split).
struct RouteDecide {
    const uint64_t *keys;           // node l's split_key maximum at l * SPLIT_KEY_STRIDE
    const SplitResult *results;     // [level nodes][F]
    SplitParams sp;
    int32_t cols;
    int64_t *node_g, *node_h;
    float2 *bounds;
    const int8_t *monotone;
    const TreeCtl *ctl;
};
// implicit_in: order_in holds launch_quantize's implicit u32 words (the
// root level of an unsampled tree).
// built_only (with decide and write_entries): of each split node only the
// child that the next level's plan builds gets its entries written, the
// child with the smaller integer hessian sum (ties left).  Only for the last
// partition before the deepest split level, whose other children's entries
// nothing reads, and only when every entry's quantised hessian is the same,
// so that the smaller hessian sum is the smaller row count, the child the
// plan builds.
hipError_t launch_route(hipStream_t s, const Shape &sh, const LevelArgs &la,
                        const uint8_t *bins_fm, const Entry *order_in, Entry *order_out,
                        const uint32_t *seg_start, uint32_t *count, const TreeOut out,
                        uint64_t *cursors, uint32_t max_blocks, bool write_entries,
                        const RoutePlan *plan = nullptr, bool implicit_in = false,
                        const RouteDecide *decide = nullptr, bool built_only = false);

// la = the level being planned (d); reads level d-1's routed counts.
hipError_t launch_plan_level(hipStream_t s, const Shape &sh, const LevelArgs &la,
                             uint32_t target_items, uint32_t min_chunk, TreeCtl *ctl,
                             const uint32_t *seg_start_prev, uint32_t *seg_start_next,
                             uint32_t *count, const uint64_t *cursors, const TreeOut out,
                             Pair *pairs, HistItem *items);

// ---------------------------------------------------------------------------
// Leaf-wise (best-first) growth (leaf_reset/leaf_init/leaf_pick_apply/
// leaf_step and the partition pipeline, Shaders.swift:656-1091).  The order
// entries live in one buffer of 2*rows: a leaf's segment sits in one half and
// its partition writes the children into the same range of the other half.
// Histograms live in slots: the smaller child of a split gets a new slot, the
// larger child inherits the parent's slot (parent - smaller, in place).
// ---------------------------------------------------------------------------

struct LWOpen {                 // an unsplit leaf of the current tree
    int32_t node;               // heap index
    uint32_t seg;               // first entry (absolute, in the double buffer)
    uint32_t count;             // rows
    int32_t depth;
    int32_t slot;               // histogram slot, -1 when not evaluated
    int32_t best_f;             // best feature, -1 when it cannot be split
    float lo, hi;               // monotone bounds of its leaf value
    int64_t g, h;               // exact quantised sums
    SplitResult best;           // best split over the allowed features
};

struct LWState {
    uint32_t done;              // no further split in this tree
    uint32_t leaves;            // current leaf count
    uint32_t open_count;        // entries used in the open list
    uint32_t next_slot;         // next free histogram slot
    uint32_t pick;              // open entry split in this step
    int32_t pick_node, pick_depth, pick_slot;   // its heap node, depth and slot
    uint32_t child0;            // open entry of the left child (right = child0 + 1)
    uint32_t eval_first;        // open entries whose best split the eval step fills
    uint32_t eval_count;
    // partition of the picked leaf
    uint32_t src;               // absolute first entry of the segment
    uint32_t dst;               // same range in the other half
    uint32_t count;             // rows in the segment
    uint32_t left;              // rows going left
    int32_t feature;
    uint32_t bin, flags;
    uint32_t mask[8];
};

struct LWArgs {
    int32_t num_leaves;         // L
    int32_t max_depth;          // D
    uint32_t rows;              // N (size of one half of the order buffer)
    uint32_t part_blocks;       // partition grid (grid-stride over PART_ENTRIES chunks)
    int32_t total_nodes;        // heap nodes per tree
    uint32_t target_items, min_chunk;
    uint32_t pad;
};

hipError_t launch_lw_init(hipStream_t s, const Shape &sh, const LWArgs &a, TreeCtl *ctl,
                          LWState *st, LWOpen *open, uint32_t *slot_seg, uint32_t *slot_count,
                          Pair *pairs, HistItem *items, const TreeOut out, bool sampled);
// the last step's evaluations (every other step's run inside the next pick)
hipError_t launch_lw_eval(hipStream_t s, const Shape &sh, const SplitParams &sp,
                          const LWState *st, LWOpen *open, const SplitResult *results,
                          const int64_t *slot_g, const int64_t *slot_h, const TreeCtl *ctl,
                          const TreeOut out);
hipError_t launch_lw_bounds(hipStream_t s, const LWState *st, const LWOpen *open,
                            float2 *bounds);
hipError_t launch_lw_pick(hipStream_t s, const Shape &sh, const SplitParams &sp, const LWArgs &a,
                          LWState *st, LWOpen *open, const SplitResult *results,
                          const int64_t *slot_g, const int64_t *slot_h, const int8_t *monotone,
                          TreeCtl *ctl, uint64_t *cursor, const TreeOut out);
// partition of the picked leaf, then (in the block that completes it) the
// plan of the children
hipError_t launch_lw_partition(hipStream_t s, const Shape &sh, const LWArgs &a, LWState *st,
                               LWOpen *open, const uint8_t *bins_fm, Entry *order,
                               uint64_t *cursor, uint32_t *slot_seg, uint32_t *slot_count,
                               TreeCtl *ctl, Pair *pairs, HistItem *items, const TreeOut out);

// Leaf-wise growth in depth rounds (trees of depth <= LWB_MAX_DEPTH).  Round r
// builds, for every depth-r leaf that can still be picked, its partition and
// its children's histograms and splits, with the level-wise kernels on a
// speculative tree; a single-block select kernel replays the best-first picks
// over the evaluated candidates and writes the picked nodes into the tree.
constexpr int LWB_MAX_DEPTH = 8;
constexpr int LWB_MAX_NODES = (1 << (LWB_MAX_DEPTH + 1)) - 1;
constexpr int LWB_MAX_LEAVES = 1 << LWB_MAX_DEPTH;
constexpr uint32_t LWB_MISSED_PICK = 2;   // TreeCtl::overflow: a pick was never expanded

struct LWBState {
    uint32_t done, leaves, open_count, pad;
    int32_t cand_f[LWB_MAX_NODES];            // best feature of an evaluated node, -1 none
    float cand_gain[LWB_MAX_NODES];           // its gain
    int32_t open[LWB_MAX_NODES];              // open-list index; -1 not open, -2 split
    int32_t olist[2 * LWB_MAX_LEAVES + 2];    // node at each open-list index
    uint32_t expanded[(LWB_MAX_NODES + 31) / 32];   // bit per node: partitioned, children built
};

struct LWBArgs {
    int32_t num_leaves;         // L <= LWB_MAX_LEAVES
    int32_t max_depth;          // D <= LWB_MAX_DEPTH
    int32_t total_nodes;        // 2^(D+1) - 1
    int32_t deep_walk;          // 1: the training walk counts the depth-D rows (the last
                                // round partitions nothing); round D zeroes their counts
};

// Round r < D: evaluate the depth-r nodes the last round built, replay the
// picks, choose the depth-r nodes to expand (their splits into spec, their
// level's partition cursors zeroed).  Round D: the remaining picks.
hipError_t launch_lwb_select(hipStream_t s, const Shape &sh, const SplitParams &sp,
                             const LWBArgs &a, int32_t round, const SplitResult *results,
                             uint32_t *count, const int64_t *node_g, const int64_t *node_h,
                             float2 *bounds, const int8_t *monotone, TreeCtl *ctl,
                             uint64_t *cursors, LWBState *st, SplitResult *cand,
                             const TreeOut spec, const TreeOut out);

// Inference.
struct ForestDev {
    const int32_t *feature;
    const float *threshold;
    const uint8_t *flags;
    const float *leaf;
    const uint32_t *mask;      // 8 words per node or NULL when no node is categorical
    int32_t num_trees;
    int32_t nodes_per_tree;
    int32_t tree_first = 0;    // walk trees tree_first, +tree_step, ... (one class of K)
    int32_t tree_step = 1;
    int32_t out_stride = 1;    // out[i * out_stride]
};
hipError_t launch_predict_forest(hipStream_t s, const ForestDev &f, const float *x,
                                 int64_t rows, int32_t data_bins, float base, float *out);
hipError_t launch_predict_binned(hipStream_t s, const uint8_t *bins_fm, int64_t rows,
                                 int32_t num_bins, int32_t max_depth, const TreeOut tree,
                                 float *preds);
// Training-row walk of a finished tree: preds += leaf (unless preds is null),
// and rows per node of the deepest level added to count[2^D - 1 ...] (unless
// count is null; with kept non-null only rows with kept[i] != 0 count).
hipError_t launch_walk_count(hipStream_t s, const uint8_t *bins_fm, int64_t rows,
                             int32_t num_bins, int32_t max_depth, const TreeOut tree,
                             float *preds, uint32_t *count, const uint8_t *kept);
// The same walk (preds required; single-output objectives) that also starts
// the next tree's gradient pass on the updated predictions: *partials pairs
// of (max |g|, max h) into gpart (at most grad_max_scratch_words() / 2), and,
// with g_out / h_out, every row's g and h.  launch_grad_max_final then takes
// the place of launch_grad_max.
hipError_t launch_walk_count_grad(hipStream_t s, const uint8_t *bins_fm, int64_t rows,
                                  int32_t num_bins, int32_t max_depth, const TreeOut tree,
                                  float *preds, uint32_t *count, const uint8_t *kept,
                                  const GradParams &gp, const float *labels,
                                  const float *weights, uint32_t *gpart, float *g_out,
                                  float *h_out, int *partials);
hipError_t launch_grad_max_final(hipStream_t s, const uint32_t *partial, int nparts,
                                 TreeCtl *ctl);

struct ShapPath {
    int32_t elem_start;   // first element
    int32_t num_elem;     // elements on the path (root first)
    int32_t uniq_start;   // first unique-feature slot
    int32_t num_uniq;     // unique features U
    double leaf;          // leaf value
};
struct ShapElem {
    int32_t node;         // global node index (tree * nodes_per_tree + node)
    int32_t feature;
    float threshold;
    uint32_t flags;       // split flags | 0x100 when the path continues left
    int32_t uniq;         // index of its unique-feature slot within the path
    int32_t pad;
};
struct ShapUniq {
    int32_t feature;
    int32_t pad;
    double zero;          // product of cover fractions along the path
};
// max_elems: the longest path's element count (1..12).  phi_global: a
// [ceil(rows/64)][cols][64] double scratch when treeshap_needs_scratch(cols)
// (wide data), else unused (may be NULL).
hipError_t launch_treeshap(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                           int32_t data_bins, const uint32_t *masks, const ShapPath *paths,
                           int32_t num_paths, int32_t max_elems, const ShapElem *elems,
                           const ShapUniq *uniq, float bias, float *out, double *phi_global);
bool treeshap_needs_scratch(int cols);

}  // namespace mbk
