// noalloc.hip — mbk_node_hist_split_noalloc: the one-node histogram build and
// split search of mbk_node_hist_split with every scratch buffer (control
// block, item list, partial histograms, node sums, default feature arrays)
// in one fixed device array, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops).  It allocates nothing,
// clears and fills its scratch with kernels (no memset nodes), and returns
// without waiting for the stream.  Every call on a GPU shares that GPU's
// array: calls that overlap on one GPU race.
#include <mutex>

#include "../../include/macboost.h"
#include "abi.hpp"
#include "core.hpp"

namespace {

// Scratch layout (byte offsets): a 64 KiB header of small buffers, then the
// partial histograms.  16 MiB in all.
constexpr size_t SCRATCH_BYTES = (size_t)16 << 20;
constexpr size_t OFF_CTL = 0;                 // mbk::TreeCtl
constexpr size_t OFF_PAIR = 256;              // one mbk::Pair
constexpr size_t OFF_SEG = 512;               // 1 u32
constexpr size_t OFF_COUNT = 576;             // 3 u32 (a depth-1 heap)
constexpr size_t OFF_COVER = 640;             // 1 f32
constexpr size_t OFF_BOUNDS = 704;            // 3 float2
constexpr size_t OFF_NODE_G = 768;            // 3 int64
constexpr size_t OFF_NODE_H = 832;            // 3 int64
constexpr size_t OFF_NO_CAT = 1024;           // [NOALLOC_MAX_COLS] u8 = 0
constexpr size_t OFF_NO_MONO = OFF_NO_CAT + 4096;
constexpr size_t OFF_ALL_FEATS = OFF_NO_MONO + 4096;
constexpr size_t OFF_ITEMS = (size_t)16 << 10;
constexpr size_t OFF_PARTIALS = (size_t)64 << 10;
constexpr int32_t NOALLOC_MAX_COLS = 4096;
constexpr size_t MAX_ITEMS = (OFF_PARTIALS - OFF_ITEMS) / sizeof(mbk::HistItem);
static_assert(sizeof(mbk::TreeCtl) <= OFF_PAIR - OFF_CTL, "control block fits");
static_assert(sizeof(mbk::Pair) <= OFF_SEG - OFF_PAIR, "pair fits");
static_assert(OFF_ALL_FEATS + NOALLOC_MAX_COLS <= OFF_ITEMS, "default arrays fit");
static_assert(OFF_PARTIALS % 256 == 0 && OFF_ITEMS % 256 == 0, "aligned regions");

}  // namespace

static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

namespace {

// The array's device address on each GPU, looked up once per device with
// that device current (the host-side name is not a device address).
std::mutex g_mu;
unsigned char *g_scratch[64] = {};

unsigned char *scratch_on(int device) {
    if (device < 0 || device >= 64) mb::internal("device index out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[device]) {
        MB_HIP(hipSetDevice(device));
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            mb::internal(std::string("hipGetSymbolAddress(scratch) failed: ") +
                         hipGetErrorString(e));
        g_scratch[device] = static_cast<unsigned char *>(p);
    }
    return g_scratch[device];
}

// Zeroes the control block and takes the caller's maxima into it; the
// default arrays become no categorical feature, no constraint, every feature.
__global__ __launch_bounds__(256) void k_noalloc_setup(unsigned char *base,
                                                       const uint32_t *__restrict__ max_gh,
                                                       int32_t cols) {
    uint32_t *ctl = reinterpret_cast<uint32_t *>(base + OFF_CTL);
    for (int k = threadIdx.x; k < (int)(sizeof(mbk::TreeCtl) / 4); k += blockDim.x)
        ctl[k] = k < 2 ? max_gh[k] : 0u;
    for (int f = threadIdx.x; f < cols; f += blockDim.x) {
        base[OFF_NO_CAT + f] = 0;
        base[OFF_NO_MONO + f] = 0;
        base[OFF_ALL_FEATS + f] = 1;
    }
}

}  // namespace

extern "C" int mbk_node_hist_split_noalloc(mbk_context *ctx, const uint8_t *bins_tiled,
                                           int64_t rows, int32_t cols, int32_t num_bins,
                                           int32_t tile_width, const uint32_t *entries, int64_t n,
                                           const uint32_t *max_gh, const uint8_t *is_cat,
                                           const int8_t *monotone, float lambda,
                                           float min_child_hess, float cat_smooth,
                                           int64_t *hist_out, mbk_split_result *results,
                                           char **err) {
    return mb::guarded(err, [&]() -> int {
        if (!ctx) mb::invalid("null kernel-seam context");
        if (num_bins < 4 || num_bins > 256) mb::invalid("numBins must be in 4...256");
        if (tile_width != 8 && tile_width != 16 && tile_width != 32 && tile_width != 64)
            mb::invalid("tile_width must be 8, 16, 32 or 64");
        if (cols < 1 || cols > NOALLOC_MAX_COLS)
            mb::invalid("mbk_node_hist_split_noalloc takes 1..4096 features");
        if (n < 0 || n > 0xFFFFFFF0LL) mb::invalid("row count out of range");
        if (rows < 0 || !bins_tiled || !entries || !max_gh || !hist_out || !results)
            mb::invalid("null or empty argument");
        mbk::Shape sh{std::max<int64_t>(rows, n), cols, num_bins, tile_width,
                      (cols + tile_width - 1) / tile_width, 0u, 0, 0, 0};
        mbk::set_hist_tiling(sh);
        const int32_t T = sh.hist_tiles;             // histogram items per row chunk
        // items of the node: the planner's budget for it, an upper bound on
        // what it plans, must fit both the item list and the partial histograms
        const size_t per_item = (size_t)sh.part_w * (size_t)num_bins * sizeof(uint64_t);
        const size_t cap = std::min(MAX_ITEMS, (SCRATCH_BYTES - OFF_PARTIALS) / per_item);
        const uint32_t target = (uint32_t)std::min<size_t>(256, cap / 2 > 0 ? cap / 2 : 1);
        const uint32_t min_chunk = 2048;
        const uint64_t items = mbk::item_budget((uint64_t)n, 1, T, target);
        if (items > cap)
            mb::invalid("node of " + std::to_string(n) + " rows needs " + std::to_string(items) +
                        " histogram items; the no-allocation scratch holds " +
                        std::to_string(cap) + " at this tile width and bin count");
        const int device = mb::context_device(ctx);
        unsigned char *base = scratch_on(device);
        MB_HIP(hipSetDevice(device));
        hipStream_t s = mb::context_stream(ctx);
        auto *ctl = reinterpret_cast<mbk::TreeCtl *>(base + OFF_CTL);
        auto *pairs = reinterpret_cast<mbk::Pair *>(base + OFF_PAIR);
        auto *seg = reinterpret_cast<uint32_t *>(base + OFF_SEG);
        auto *count = reinterpret_cast<uint32_t *>(base + OFF_COUNT);
        auto *cover = reinterpret_cast<float *>(base + OFF_COVER);
        auto *bounds = reinterpret_cast<float2 *>(base + OFF_BOUNDS);
        auto *node_g = reinterpret_cast<int64_t *>(base + OFF_NODE_G);
        auto *node_h = reinterpret_cast<int64_t *>(base + OFF_NODE_H);
        auto *items_d = reinterpret_cast<mbk::HistItem *>(base + OFF_ITEMS);
        auto *partials = reinterpret_cast<uint64_t *>(base + OFF_PARTIALS);
        const auto *no_cat = reinterpret_cast<const uint8_t *>(base + OFF_NO_CAT);
        const auto *no_mono = reinterpret_cast<const int8_t *>(base + OFF_NO_MONO);
        const auto *all_feats = reinterpret_cast<const uint8_t *>(base + OFF_ALL_FEATS);
        sh.item_cap = (uint32_t)cap;
        const mbk::SplitParams sp{lambda, min_child_hess, 0.0f, cat_smooth, 0.1f, 1};
        hipLaunchKernelGGL(k_noalloc_setup, dim3(1), dim3(256), 0, s, base, max_gh, cols);
        MB_HIP(hipGetLastError());
        const mbk::RootPlan rp{sh,      (uint32_t)n, target, min_chunk, 0u,     ctl,
                               seg,     count,       pairs,  items_d,   cover,  bounds,
                               -INFINITY, INFINITY};
        MB_HIP(mbk::launch_plan_root(s, rp));
        MB_HIP(mbk::launch_hist(s, sh, bins_tiled, reinterpret_cast<const mbk::Entry *>(entries),
                                items_d, ctl, partials, (int)std::max<uint32_t>(target, 1)));
        MB_HIP(mbk::launch_split(s, sh, sp, pairs, 1, partials, node_g, hist_out,
                                 is_cat ? is_cat : no_cat, monotone ? monotone : no_mono,
                                 all_feats, ctl, count, node_g, node_h, 0,
                                 reinterpret_cast<mbk::SplitResult *>(results)));
        return 0;
    }, -1);
}
