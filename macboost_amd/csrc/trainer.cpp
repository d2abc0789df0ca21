// trainer.cpp — the training driver: fitImpl (Booster.swift:445-1701) restated
// for one MI355X.  The raw matrix is uploaded once; quantile edges
// (Binner.swift:25-56) and bins are computed on the device, and every tree is a fixed sequence of
// kernels on one HIP stream with all split decisions kept on the device; the
// host touches the stream again only to read finished trees (or, with a
// validation set, the per-iteration metric).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <exception>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "core.hpp"

namespace mb {

int host_threads() {
    unsigned n = std::thread::hardware_concurrency();
    if (n == 0) n = 1;
    if (n > 16) n = 16;
    return (int)n;
}

// Host worker threads for the block loops, started once (starting threads
// per loop costs more than the loops over a few million labels).  A loop
// runs on its calling thread and on idle workers, so loops from several
// threads progress together.  The pool lives until the process ends.
namespace {
class HostPool {
public:
    static HostPool &get() {
        static HostPool *pool = new HostPool(host_threads() - 1);
        return *pool;
    }
    // fn(k) for every k in [0, count); returns once all have returned.  fn
    // must not throw.
    void run(int64_t count, const std::function<void(int64_t)> &fn) {
        if (count <= 0) return;
        if (count == 1 || threads_.empty()) {
            for (int64_t k = 0; k < count; ++k) fn(k);
            return;
        }
        auto job = std::make_shared<Job>();
        job->count = count;
        job->fn = &fn;
        {
            std::lock_guard<std::mutex> lk(mu_);
            jobs_.push_back(job);
        }
        cv_.notify_all();
        work_on(*job);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return job->finished.load() == job->count; });
        jobs_.erase(std::find(jobs_.begin(), jobs_.end(), job));
    }

private:
    struct Job {
        int64_t count = 0;
        const std::function<void(int64_t)> *fn = nullptr;
        std::atomic<int64_t> next{0}, finished{0};
    };
    explicit HostPool(int workers) {
        for (int k = 0; k < workers; ++k) threads_.emplace_back([this] { worker(); });
    }
    void work_on(Job &j) {
        for (int64_t k = j.next++; k < j.count; k = j.next++) {
            (*j.fn)(k);
            if (++j.finished == j.count) {
                std::lock_guard<std::mutex> lk(mu_);
                done_cv_.notify_all();
            }
        }
    }
    std::shared_ptr<Job> open_job() {            // with mu_ held
        for (auto &j : jobs_)
            if (j->next.load() < j->count) return j;
        return nullptr;
    }
    void worker() {
        for (;;) {
            std::shared_ptr<Job> j;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return (j = open_job()) != nullptr; });
            }
            work_on(*j);
        }
    }
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    std::vector<std::shared_ptr<Job>> jobs_;
    std::vector<std::thread> threads_;
};
}  // namespace

// Runs fn(begin, end) over [0, n) in blocks of `block` items on the host
// pool (block b is [b*block, min(n, (b+1)*block))), and waits; fn must only
// write what its own block owns.
template <typename Fn>
static void parallel_blocks(int64_t n, int64_t block, Fn fn) {
    const int64_t nblocks = (n + block - 1) / block;
    const std::function<void(int64_t)> f = [&](int64_t b) {
        fn(b * block, std::min(n, (b + 1) * block));
    };
    HostPool::get().run(nblocks, f);
}

// Rows per block of the sums over every row (base score): a block's rows
// are summed in double in the order of the device's k_label_stats (lane l of
// 64 adds rows l, l + 64, ... in order, then lane l adds lane l + s for
// s = 32, 16, ..., 1), then the block sums in block order, so the result does
// not depend on how blocks are spread over threads, or on where they run.
constexpr int64_t SUM_BLOCK = 65536;

// Per-block double sums of two accumulators that add(i, a, b) updates, into
// s1[k], s2[k] for block k (rows [k*SUM_BLOCK, ...)).
template <typename Add>
static void sum_blocks(int64_t n, double *s1, double *s2, Add add) {
    parallel_blocks(n, SUM_BLOCK, [&](int64_t a, int64_t b) {
        double x[64] = {}, y[64] = {};
        for (int64_t r = a; r < b; r += 64) {
            const int m = (int)std::min<int64_t>(64, b - r);
            for (int l = 0; l < m; ++l) add(r + l, x[l], y[l]);
        }
        for (int st = 32; st >= 1; st >>= 1)
            for (int l = 0; l < st; ++l) {
                x[l] += x[l + st];
                y[l] += y[l + st];
            }
        s1[(size_t)(a / SUM_BLOCK)] = x[0];
        s2[(size_t)(a / SUM_BLOCK)] = y[0];
    });
}

static double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

std::string swift_float(float v) {
    if (std::isnan(v)) return "nan";
    if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
    char buf[64];
    if (v == std::floor(v) && std::fabs(v) < 1e16f) {
        std::snprintf(buf, sizeof buf, "%.1f", (double)v);
        return buf;
    }
    std::snprintf(buf, sizeof buf, "%.9g", (double)v);
    // shortest representation that round-trips
    for (int prec = 1; prec <= 9; ++prec) {
        char b2[64];
        std::snprintf(b2, sizeof b2, "%.*g", prec, (double)v);
        if (std::strtof(b2, nullptr) == v) return b2;
    }
    return buf;
}

// ---------------------------------------------------------------------------
// Device memory cache (DevBuf::pooled)
// ---------------------------------------------------------------------------

namespace {
struct CachedBlock {
    void *p;
    size_t bytes;
    int device;
    uint64_t tick;
};
std::mutex g_pool_mu;
std::vector<CachedBlock> g_pool;
size_t g_pool_bytes[64] = {};
size_t g_pool_limit[64] = {};
uint64_t g_pool_tick = 0;

size_t pool_limit(int device) {             // with g_pool_mu held
    if (device < 0 || device >= 64) return 0;
    if (!g_pool_limit[device]) {
        size_t free_b = 0, total_b = 0;
        if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) total_b = 0;
        g_pool_limit[device] = total_b / 2 + 1;
    }
    return g_pool_limit[device];
}
}  // namespace

hipError_t malloc_or_trim(void **p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        pool_trim();
        e = hipMalloc(p, bytes);
    }
    return e;
}

void *pool_alloc(size_t bytes, int *device) {
    int dev = 0;
    MB_HIP(hipGetDevice(&dev));
    *device = dev;
    {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        for (size_t k = 0; k < g_pool.size(); ++k) {
            if (g_pool[k].device == dev && g_pool[k].bytes == bytes) {
                void *p = g_pool[k].p;
                g_pool[k] = g_pool.back();
                g_pool.pop_back();
                if (dev >= 0 && dev < 64) g_pool_bytes[dev] -= bytes;
                return p;
            }
        }
    }
    void *p = nullptr;
    MB_HIP(malloc_or_trim(&p, bytes));
    return p;
}

void pool_free(void *p, size_t bytes, int device) {
    std::vector<void *> evict;
    {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        const size_t limit = pool_limit(device);
        if (device < 0 || device >= 64 || bytes > limit) {
            evict.push_back(p);
        } else {
            g_pool.push_back({p, bytes, device, ++g_pool_tick});
            g_pool_bytes[device] += bytes;
            while (g_pool_bytes[device] > limit) {   // oldest blocks of this device first
                size_t oldest = g_pool.size();
                for (size_t k = 0; k < g_pool.size(); ++k)
                    if (g_pool[k].device == device &&
                        (oldest == g_pool.size() || g_pool[k].tick < g_pool[oldest].tick))
                        oldest = k;
                evict.push_back(g_pool[oldest].p);
                g_pool_bytes[device] -= g_pool[oldest].bytes;
                g_pool[oldest] = g_pool.back();
                g_pool.pop_back();
            }
        }
    }
    for (void *q : evict) (void)hipFree(q);
}

void pool_trim() {
    std::vector<CachedBlock> all;
    {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        all.swap(g_pool);
        for (size_t &b : g_pool_bytes) b = 0;
    }
    for (const CachedBlock &b : all) (void)hipFree(b.p);
}

Device::Device(int device_id) : id(device_id) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device_id)
        throw Error("No HIP GPU available");
    MB_HIP(hipSetDevice(device_id));
    MB_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    MB_HIP(hipStreamCreateWithFlags(&copy_stream, hipStreamNonBlocking));
    // the CU count, looked up once per device (a properties query costs ~1 ms)
    static std::mutex mu;
    static int cus[64] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (device_id >= 64 || !cus[device_id]) {
        int n = 0;
        MB_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device_id));
        if (device_id >= 64) { num_cus = n; return; }
        cus[device_id] = n;
    }
    num_cus = cus[device_id];
}

Device::~Device() {
    if (stream) (void)hipStreamDestroy(stream);
    if (copy_stream) (void)hipStreamDestroy(copy_stream);
}

// Devices whose owners ended, kept with their streams for the next owner
// (creating a stream costs about a millisecond).  The list is never torn
// down: its streams live until the process ends.
namespace {
std::mutex g_dev_mu;
std::vector<Device *> *g_dev_free = new std::vector<Device *>();
}  // namespace

std::unique_ptr<Device> acquire_device(int device_id) {
    {
        std::lock_guard<std::mutex> lock(g_dev_mu);
        for (size_t k = 0; k < g_dev_free->size(); ++k) {
            if ((*g_dev_free)[k]->id == device_id) {
                Device *d = (*g_dev_free)[k];
                (*g_dev_free)[k] = g_dev_free->back();
                g_dev_free->pop_back();
                MB_HIP(hipSetDevice(device_id));
                return std::unique_ptr<Device>(d);
            }
        }
    }
    return std::make_unique<Device>(device_id);
}

void release_device(std::unique_ptr<Device> d) {
    if (!d) return;
    std::lock_guard<std::mutex> lock(g_dev_mu);
    if (g_dev_free->size() < 16) g_dev_free->push_back(d.release());
}

// Timing events for the profiled histogram launches, kept for reuse (a fit
// records two per launch; creating them costs microseconds each).
namespace {
std::mutex g_ev_mu;
std::vector<hipEvent_t> *g_ev_free = new std::vector<hipEvent_t>();

hipEvent_t acquire_event() {
    {
        std::lock_guard<std::mutex> lock(g_ev_mu);
        if (!g_ev_free->empty()) {
            hipEvent_t e = g_ev_free->back();
            g_ev_free->pop_back();
            return e;
        }
    }
    hipEvent_t e = nullptr;
    MB_HIP(hipEventCreate(&e));
    return e;
}

void release_event(hipEvent_t e) {
    if (!e) return;
    std::lock_guard<std::mutex> lock(g_ev_mu);
    g_ev_free->push_back(e);
}
}  // namespace

// ---------------------------------------------------------------------------
// Host -> device upload of large pageable buffers: two pinned staging buffers,
// each filled by a few host threads while the other one's DMA is in flight.
// Measured on MI355X for 4 GB: 55 GB/s against 29 GB/s for one pageable copy.
// The pipeline runs on across calls: a buffer is refilled once its own last
// DMA is done (an event per buffer), so back-to-back uploads (a matrix sent
// one feature tile at a time) keep the link busy between them, and an upload
// returns as soon as its source has been read.
// ---------------------------------------------------------------------------

namespace {
constexpr size_t STAGE_CHUNK = (size_t)64 << 20;
constexpr size_t STAGE_MIN = (size_t)4 << 20;     // smaller copies go straight from pageable memory
constexpr size_t STAGE_FIRST = (size_t)8 << 20;   // first piece when no DMA is in flight

struct Staging {
    std::mutex m;
    char *buf[2] = {nullptr, nullptr};   // pinned; kept for the process's lifetime
    hipEvent_t done[2] = {nullptr, nullptr};   // each buffer's last DMA, while busy
    bool busy[2] = {false, false};
    int device = -1;                     // the events' device
    unsigned next = 0;                   // the buffer the next piece fills
};

Staging &staging() {
    static Staging st;
    return st;
}

void parallel_copy(char *dst, const char *src, size_t n, unsigned threads) {
    const size_t per = (n + threads - 1) / threads;
    const std::function<void(int64_t)> f = [&](int64_t t) {
        const size_t a = (size_t)t * per, b = std::min(n, a + per);
        if (a < b) std::memcpy(dst + a, src + a, b - a);
    };
    HostPool::get().run((int64_t)threads, f);
}

// Waits until buffer b's last DMA has completed.
void staging_wait(Staging &st, unsigned b) {
    if (st.busy[b]) {
        MB_HIP(hipEventSynchronize(st.done[b]));
        st.busy[b] = false;
    }
}

// Both staging buffers, allocated on first use, and their events on the
// current device (moving to another device first drains the pipeline); false
// if pinned memory cannot be had (the caller then makes one pageable copy).
// Called with st.m held.
bool staging_ready(Staging &st) {
    for (char *&b : st.buf)
        if (!b && hipHostMalloc(reinterpret_cast<void **>(&b), STAGE_CHUNK,
                                hipHostMallocPortable) != hipSuccess) {
            b = nullptr;
            (void)hipGetLastError();
        }
    if (!st.buf[0] || !st.buf[1]) return false;
    int dev = 0;
    MB_HIP(hipGetDevice(&dev));
    if (st.device != dev) {
        for (unsigned b = 0; b < 2; ++b) {
            staging_wait(st, b);
            if (st.done[b]) (void)hipEventDestroy(st.done[b]);
            st.done[b] = nullptr;
            MB_HIP(hipEventCreateWithFlags(&st.done[b], hipEventDisableTiming));
        }
        st.device = dev;
    }
    return true;
}

unsigned copy_threads() {
    return std::max(1u, std::min(8u, std::thread::hardware_concurrency() / 2));
}
}  // namespace

void upload(void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (bytes < STAGE_MIN) {
        MB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
        return;
    }
    Staging &st = staging();
    std::lock_guard<std::mutex> lock(st.m);
    if (!staging_ready(st)) {                        // no pinned memory: one pageable copy
        MB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
        return;
    }
    const unsigned threads = copy_threads();
    const char *from = static_cast<const char *>(src);
    char *to = static_cast<char *>(dst);
    // pieces of at least a quarter of the copy (so a host fill overlaps the
    // DMA of another), at most a buffer; with no DMA in flight the first
    // pieces start small and double, so the link starts after a short fill
    const size_t full = std::min(STAGE_CHUNK, std::max(STAGE_MIN, (bytes + 3) / 4));
    size_t piece = st.busy[0] || st.busy[1] ? full : std::min(full, STAGE_FIRST);
    for (size_t off = 0; off < bytes;) {
        const unsigned b = st.next;
        st.next ^= 1u;
        const size_t n = std::min(piece, bytes - off);
        staging_wait(st, b);                         // its previous DMA is done
        parallel_copy(st.buf[b], from + off, n, threads);
        MB_HIP(hipMemcpyAsync(to + off, st.buf[b], n, hipMemcpyHostToDevice, s));
        MB_HIP(hipEventRecord(st.done[b], s));
        st.busy[b] = true;
        off += n;
        piece = std::min(full, 2 * piece);
    }
}

void download(void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (bytes < STAGE_CHUNK) {
        MB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
        MB_HIP(hipStreamSynchronize(s));
        return;
    }
    Staging &st = staging();
    std::lock_guard<std::mutex> lock(st.m);
    if (!staging_ready(st)) {
        MB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
        MB_HIP(hipStreamSynchronize(s));
        return;
    }
    const unsigned threads = copy_threads();
    // the uploads' DMAs out of the buffers first
    staging_wait(st, 0);
    staging_wait(st, 1);
    hipEvent_t ev[2] = {nullptr, nullptr};
    MB_HIP(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming));
    MB_HIP(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming));
    const char *from = static_cast<const char *>(src);
    char *to = static_cast<char *>(dst);
    const size_t nchunks = (bytes + STAGE_CHUNK - 1) / STAGE_CHUNK;
    auto issue = [&](size_t k) {                     // DMA of chunk k into buffer k % 2
        const size_t off = k * STAGE_CHUNK, n = std::min(STAGE_CHUNK, bytes - off);
        MB_HIP(hipMemcpyAsync(st.buf[k & 1], from + off, n, hipMemcpyDeviceToHost, s));
        MB_HIP(hipEventRecord(ev[k & 1], s));
    };
    issue(0);
    if (nchunks > 1) issue(1);
    for (size_t k = 0; k < nchunks; ++k) {
        const size_t off = k * STAGE_CHUNK, n = std::min(STAGE_CHUNK, bytes - off);
        MB_HIP(hipEventSynchronize(ev[k & 1]));
        parallel_copy(to + off, st.buf[k & 1], n, threads);
        if (k + 2 < nchunks) issue(k + 2);           // the buffer is free again
    }
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
}

// ---------------------------------------------------------------------------

struct Trainer {
    Params p;                        // effective (a dataset's bins and categoricals)
    Params user_params;              // as given; stored in the model
    bool has_feature_names = false;
    std::vector<std::string> feature_names;
    std::unique_ptr<Device> dev;
    mbk::Shape sh{};
    mbk::Shape sh_root{};          // the unsampled root's histogram shape (its planar copy)
    mbk::SplitParams sp{};
    mbk::GradParams gp{};
    int D = 6, total_nodes = 0, max_level_nodes = 1;
    int64_t rows = 0;
    int cols = 0, nb = 256;
    std::vector<float> edges;
    std::vector<uint8_t> is_cat_h, mask_base;
    std::vector<int8_t> mono_h;
    std::vector<float> labels_h, vlabels_h;
    bool has_weights = false, has_valid = false, has_cats = false;
    int64_t vrows = 0;
    float base = 0.0f;

    DevBuf<uint8_t> bins_tiled, bins_fm, vbins_fm;
    DevBuf<uint8_t> bins_root;      // planar copy of bins_tiled for the root pass
    bool has_root_copy = false;
    mbk::HistLayout root_layout{};
    DevBuf<float> labels, weights, preds, vpreds;
    DevBuf<uint8_t> is_cat, feat_mask;
    DevBuf<int8_t> mono;
    DevBuf<mbk::Entry> order_a, order_b;
    DevBuf<uint32_t> gmax_part, goss_buckets;
    // a sampled tree's gradients (g, h of every row) and its kept rows'
    // weighted hessians
    DevBuf<float> samp_g, samp_h, samp_h_kept;
    // kept[i] of a sampled level-wise tree, for the terminal walk's counts
    DevBuf<uint8_t> kept;
    bool labels_ready = false;      // labels already uploaded during the setup
    bool weights_ready = false;     // weights too
    // gradient-maxima partials the last tree's walk left for the next tree
    // (0: the next tree runs its own gradient pass)
    int walk_gparts = 0;
    bool kept_walk = false;
    DevBuf<uint64_t> route_cursor;
    // level-wise: each node's best (gain, feature) key from the split search,
    // for decisions made inside the next partition
    DevBuf<uint64_t> split_keys;
    DevBuf<uint32_t> route_done;    // the partition's finished-workgroup count (zero between launches)
    uint32_t route_grid = 1;
    DevBuf<uint64_t> partials;
    DevBuf<mbk::HistItem> items;
    DevBuf<mbk::Pair> pairs;
    DevBuf<int64_t> hist_a, hist_b;
    DevBuf<mbk::SplitResult> results;
    DevBuf<uint32_t> count, seg_a, seg_b;
    DevBuf<int64_t> node_g, node_h;
    DevBuf<float2> bounds;
    DevBuf<mbk::TreeCtl> ctl, ctl_hist;
    int ctl_pending = -1;           // tree whose ctl is not yet copied into ctl_hist
    // a finished tree's deepest covers (and empty leaves), written by the next
    // tree's root pass or at the end of the grow call
    mbk::PendingFixup fix_pending{};
    int fix_tree = -1;             // the tree fix_pending belongs to (its out is rebuilt on use:
                                   // ensure_capacity may have moved the model arrays since)
    // warm start: the init model's trees prefix the ensemble and its raw
    // scores seed preds (Booster.swift:849-866, :890-891)
    std::vector<Tree> init_trees;
    std::vector<float> seed_train, seed_valid;     // raw scores [rows][K], until uploaded
    // multiclass: K trees per round, preds [K][rows]; tree t fits class t % K
    int K = 1;
    std::vector<float> base_scores;
    float *preds_cur = nullptr, *vpreds_cur = nullptr;   // the current tree's class
    // leaf renewal (L1 / quantile objectives)
    bool renewal = false;
    float renewal_q = 0.5f;
    DevBuf<uint32_t> rn_leaf, rn_keys, rn_seg, rn_cnt, rn_off, rn_cursor;
    DevBuf<float> rn_delta;
    // leaf-wise growth
    bool leafwise = false;
    mbk::LWArgs lw{};
    DevBuf<mbk::LWState> lw_state;
    DevBuf<mbk::LWOpen> lw_open;
    // leaf-wise growth in depth rounds: the select state, the evaluated
    // candidates per node and the speculative tree the partition reads
    bool lw_rounds = false;
    mbk::LWBArgs lwb{};
    DevBuf<mbk::LWBState> lwb_state;
    DevBuf<mbk::SplitResult> lwb_cand;
    DevBuf<mbk::NodeSplit> spec_split;
    DevBuf<float> spec_cover;
    DevBuf<uint32_t> spec_mask;
    DevBuf<mbk::NodeSplit> m_split;
    DevBuf<float> m_leaf, m_gain, m_cover;
    DevBuf<uint32_t> m_mask;
    int capacity = 0, grown = 0;
    int hist_grid = 256, target_items = 512, min_chunk = 2048;
    std::vector<std::vector<uint8_t>> tree_masks;

    bool profiling = false;
    int prof_first_tree = 0;
    int prof_every = 1;             // time the histogram launches of every k-th tree
    bool prof_tree(int tree) const {
        return profiling && (tree - prof_first_tree) % prof_every == 0;
    }
    // level `next`'s planning, run by the partition's last workgroup
    mbk::RoutePlan route_plan(const mbk::LevelArgs &next, uint32_t *seg_next) {
        return mbk::RoutePlan{next,        (uint32_t)target_items, (uint32_t)min_chunk,
                              ctl.ptr,     seg_next,               pairs.ptr,
                              items.ptr,   route_done.ptr};
    }
    struct HistEvent { hipEvent_t start, end; int level; };
    std::vector<HistEvent> events;
    int64_t prof_launches = 0;
    double prof_ms = 0.0;
    double prof_level_ms[16] = {};

    // metrics / early stopping (Booster.swift:1650-1696)
    int best_iter = 0;
    float best_metric = 0.0f;
    int stale = 0;
    bool stopped = false;
    std::vector<float> eval_history;
    std::vector<std::string> warnings;
    double t_edges = 0.0, t_bin = 0.0;

    Trainer() {
        // Every buffer of a fit comes from the device memory cache: a fit of
        // the same shape finds them there (the model arrays are taken from it
        // as they grow).
        for (DevBuf<uint8_t> *b : {&bins_tiled, &bins_fm, &vbins_fm, &bins_root, &kept, &is_cat,
                                   &feat_mask})
            b->pooled = true;
        for (DevBuf<float> *b : {&labels, &weights, &preds, &vpreds, &samp_g, &samp_h,
                                 &samp_h_kept, &rn_delta, &spec_cover})
            b->pooled = true;
        for (DevBuf<uint32_t> *b : {&gmax_part, &goss_buckets, &count, &seg_a, &seg_b, &rn_leaf,
                                    &rn_keys, &rn_seg, &rn_cnt, &rn_off, &rn_cursor, &spec_mask})
            b->pooled = true;
        for (DevBuf<int64_t> *b : {&hist_a, &hist_b, &node_g, &node_h}) b->pooled = true;
        order_a.pooled = order_b.pooled = partials.pooled = items.pooled = true;
        mono.pooled = route_cursor.pooled = pairs.pooled = results.pooled = true;
        route_done.pooled = true;
        bounds.pooled = ctl.pooled = true;
        lw_state.pooled = lw_open.pooled = lwb_state.pooled = lwb_cand.pooled = true;
        spec_split.pooled = true;
    }

    ~Trainer() {
        // cached blocks and the device's streams must be idle when handed back
        if (dev) {
            if (dev->stream) (void)hipStreamSynchronize(dev->stream);
            if (dev->copy_stream) (void)hipStreamSynchronize(dev->copy_stream);
        }
        for (auto &e : events) { release_event(e.start); release_event(e.end); }
        release_device(std::move(dev));
    }

    mbk::TreeOut tree_out(int t) {
        mbk::TreeOut o;
        size_t base_n = (size_t)t * total_nodes;
        o.split = m_split.ptr + base_n;
        o.leaf = m_leaf.ptr + base_n;
        o.gain = m_gain.ptr + base_n;
        o.cover = m_cover.ptr + base_n;
        o.mask = m_mask.ptr + base_n * 8;
        return o;
    }

    void ensure_capacity(int n) {
        if (n <= capacity) return;
        int cap = std::max(n, capacity * 2);
        auto grow = [&](auto &buf, size_t per_tree) {
            using T = typename std::remove_reference<decltype(*buf.ptr)>::type;
            DevBuf<T> nbuf;                             // the old block goes after the sync
            nbuf.pooled = true;
            nbuf.alloc((size_t)cap * per_tree);
            MB_HIP(hipMemsetAsync(nbuf.ptr, 0, nbuf.bytes(), dev->stream));
            if (buf.ptr && capacity)
                MB_HIP(hipMemcpyAsync(nbuf.ptr, buf.ptr, (size_t)capacity * per_tree * sizeof(T),
                                      hipMemcpyDeviceToDevice, dev->stream));
            MB_HIP(hipStreamSynchronize(dev->stream));
            buf = std::move(nbuf);
        };
        grow(m_split, total_nodes);
        grow(m_leaf, total_nodes);
        grow(m_gain, total_nodes);
        grow(m_cover, total_nodes);
        grow(m_mask, (size_t)total_nodes * 8);
        grow(ctl_hist, 1);
        capacity = cap;
    }
};

// The check of one label; throws the reference's message for row i.
static void check_label(const Params &p, const float *y, int64_t i) {
    const bool logistic = p.objective == OBJ_LOGISTIC;
    const bool nonneg = p.objective == OBJ_POISSON || p.objective == OBJ_TWEEDIE;
    {
        float v = y[i];
        if (!std::isfinite(v))
            invalid("label at row " + std::to_string(i) + " is " + swift_float(v) +
                    "; labels must be finite");
        if (logistic && v != 0.0f && v != 1.0f)
            invalid("label at row " + std::to_string(i) + " is " + swift_float(v) +
                    "; binary objective requires labels in {0, 1}");
        if (nonneg && v < 0.0f)
            invalid("label at row " + std::to_string(i) + " is " + swift_float(v) + "; " +
                    objective_name(p.objective) + " requires labels >= 0");
        if (p.objective == OBJ_MULTICLASS) {
            const float r = std::nearbyint(v);
            if (r != v || r < 0.0f || (int64_t)r >= p.num_classes)
                invalid("label at row " + std::to_string(i) + " is " + swift_float(v) +
                        "; multiclass requires integer labels in 0..<" +
                        std::to_string(p.num_classes));
        }
    }
}

// First row in [a, b) whose label check_label rejects, or -1: the same
// rules as a plain predicate, so the scan runs without calls.
template <int OBJ>
static int64_t first_bad_label(const float *y, int64_t a, int64_t b, int num_classes) {
    for (int64_t i = a; i < b; ++i) {
        const float v = y[i];
        bool ok = std::isfinite(v);
        if (OBJ == OBJ_LOGISTIC) ok = ok && (v == 0.0f || v == 1.0f);
        if (OBJ == OBJ_POISSON || OBJ == OBJ_TWEEDIE) ok = ok && v >= 0.0f;
        if (OBJ == OBJ_MULTICLASS) {
            const float r = std::nearbyint(v);
            ok = ok && r == v && r >= 0.0f && (int64_t)r < num_classes;
        }
        if (!ok) return i;
    }
    return -1;
}

// Labels (Booster.swift:1724-1765), scanned in blocks on the host threads;
// the first offending row over all blocks gets the message.
static void validate_labels(const Params &p, const float *y, int64_t n) {
    const int64_t block = 1 << 18;
    const int64_t nblocks = (n + block - 1) / block;
    std::vector<int64_t> first((size_t)nblocks, -1);
    const int obj = p.objective, nc = p.num_classes;
    parallel_blocks(n, block, [&](int64_t a, int64_t b) {
        int64_t f;
        switch (obj) {
        case OBJ_LOGISTIC: f = first_bad_label<OBJ_LOGISTIC>(y, a, b, nc); break;
        case OBJ_POISSON: f = first_bad_label<OBJ_POISSON>(y, a, b, nc); break;
        case OBJ_TWEEDIE: f = first_bad_label<OBJ_TWEEDIE>(y, a, b, nc); break;
        case OBJ_MULTICLASS: f = first_bad_label<OBJ_MULTICLASS>(y, a, b, nc); break;
        default: f = first_bad_label<-1>(y, a, b, nc); break;
        }
        first[(size_t)(a / block)] = f;
    });
    for (int64_t f : first)
        if (f >= 0) check_label(p, y, f);
}

void validate_label_values(const Params &p, const float *y, int64_t n) { validate_labels(p, y, n); }

// multiclassLogloss (Booster.swift:1828-1841) over preds [K][n].
static float multiclass_logloss(const float *pred, const float *y, int64_t n, int K) {
    double s = 0;
    for (int64_t i = 0; i < n; ++i) {
        double m = -INFINITY;
        for (int k = 0; k < K; ++k) m = std::max(m, (double)pred[(int64_t)k * n + i]);
        double sum = 0;
        for (int k = 0; k < K; ++k) sum += std::exp((double)pred[(int64_t)k * n + i] - m);
        const int c = (int)y[i];
        s -= (double)pred[(int64_t)c * n + i] - m - std::log(sum);
    }
    return (float)(s / (double)n);
}

void validate_categoricals(const Params &p, const float *x, int64_t rows, int64_t cols,
                                  int64_t rs, int64_t cs) {          // :1810-1826
    const int data_bins = p.num_bins - 1;
    for (int f : p.categorical) {
        if (f < 0 || f >= cols)
            internal("categorical feature index " + std::to_string(f) + " out of range");
        for (int64_t i = 0; i < rows; ++i) {
            float v = x[i * rs + (int64_t)f * cs];
            if (std::isnan(v)) continue;
            float c = std::nearbyint(v);
            if (!(c >= 0.0f) || !std::isfinite(c) || (int64_t)c >= data_bins)
                throw Error("Categorical feature " + std::to_string(f) + " has value " +
                            swift_float(v) + "; expected integer ids in 0..<" +
                            std::to_string(data_bins) + " or NaN");
        }
    }
}

// Target-leakage guard (Booster.swift:1771-1808).  On every
// max(1, rows / 4096)-th row (at least 50 of them), each feature's finite
// values are correlated with the label (Pearson r, the label centred on its
// mean over all sampled rows); |r| > 0.999 over at least 50 finite values
// adds a warning to `out` (and prints it when verbose).
static void check_leakage(bool verbose, const float *x, int64_t rows, int64_t cols, int64_t rs,
                          int64_t cs, const float *y, std::vector<std::string> &out) {
    const int64_t step = std::max<int64_t>(1, rows / 4096);
    const int64_t m = (rows + step - 1) / step;          // sampled rows
    if (m < 50) return;
    double ysum = 0;
    for (int64_t k = 0; k < m; ++k) ysum += (double)y[k * step];
    const double ymean = ysum / (double)m;
    std::vector<double> dy((size_t)m);
    for (int64_t k = 0; k < m; ++k) dy[(size_t)k] = (double)y[k * step] - ymean;
    std::vector<double> xv;                              // the column's finite samples
    std::vector<int64_t> slot;                           // ... and where they were sampled
    for (int64_t f = 0; f < cols; ++f) {
        xv.clear();
        slot.clear();
        for (int64_t k = 0; k < m; ++k) {
            const float v = x[k * step * rs + f * cs];
            if (!std::isfinite(v)) continue;
            xv.push_back((double)v);
            slot.push_back(k);
        }
        if (xv.size() < 50) continue;
        double xsum = 0;
        for (double v : xv) xsum += v;
        const double xmean = xsum / (double)xv.size();
        double cxy = 0, cxx = 0, cyy = 0;
        for (size_t j = 0; j < xv.size(); ++j) {
            const double a = xv[j] - xmean, b = dy[(size_t)slot[j]];
            cxy += a * b;
            cxx += a * a;
            cyy += b * b;
        }
        if (!(cxx > 0 && cyy > 0)) continue;
        const double r = std::fabs(cxy / (std::sqrt(cxx) * std::sqrt(cyy)));
        if (!(r > 0.999)) continue;
        char msg[256];
        std::snprintf(msg, sizeof msg,
                      "[MacBoost] [Warning] feature %lld correlates with the label at "
                      "|r|=%.4f on a subsample — possible target leakage (is the label or a "
                      "prediction included in X?)",
                      (long long)f, r);
        out.push_back(msg);
        if (verbose) std::printf("%s\n", msg);
    }
}

// The base score from the two sums over every row (baseScore,
// Booster.swift:798-830): logistic, the log odds of the (scale_pos_weight
// weighted) positive share; otherwise the weighted label mean (its log for
// Poisson and Tweedie).
static float base_from_sums(const Params &p, double s1, double s2) {
    if (p.objective == OBJ_LOGISTIC) {
        float pr = (float)(s1 / std::max(s2, 1e-12));
        pr = std::min(std::max(pr, 1e-6f), 1.0f - 1e-6f);
        return std::log(pr / (1.0f - pr));
    }
    const float m = s2 > 0 ? (float)(s1 / s2) : 0.0f;
    if (p.objective == OBJ_POISSON || p.objective == OBJ_TWEEDIE) {
        if (!(m > 0)) invalid(objective_name(p.objective) + " requires a positive label mean");
        return std::log(m);
    }
    return m;
}

// Objectives whose base score is a sum over every row (the device computes
// it with the label checks, k_label_stats); the others take a subsample
// quantile or class counts on the host.
static bool sums_base(const Params &p) {
    return p.objective != OBJ_MAE && p.objective != OBJ_QUANTILE &&
           p.objective != OBJ_MULTICLASS;
}

static float base_score(const Params &p, const float *y, const float *w, int64_t n) {
    if (p.objective == OBJ_MAE || p.objective == OBJ_QUANTILE) {   // :786-794, :798-801
        const float q = p.objective == OBJ_MAE ? 0.5f : p.alpha;
        const int64_t step = std::max<int64_t>(1, n / 200000);
        std::vector<float> s;
        for (int64_t i = 0; i < n; i += step) s.push_back(y[i]);
        std::sort(s.begin(), s.end());
        const int64_t idx = std::min<int64_t>((int64_t)s.size() - 1,
                                              (int64_t)((float)s.size() * q));
        return s[(size_t)idx];
    }
    const int64_t nblocks = (n + SUM_BLOCK - 1) / SUM_BLOCK;
    std::vector<double> s1((size_t)nblocks, 0.0), s2((size_t)nblocks, 0.0);
    if (p.objective == OBJ_LOGISTIC) {                     // :802-830
        const double spw = (double)p.scale_pos_weight;
        sum_blocks(n, s1.data(), s2.data(), [&](int64_t i, double &pos, double &tot) {
            const double wi = w ? (double)w[i] : 1.0;
            if (y[i] > 0.5f) { pos += wi * spw; tot += wi * spw; } else tot += wi;
        });
    } else {
        sum_blocks(n, s1.data(), s2.data(), [&](int64_t i, double &num, double &den) {
            const double wi = w ? (double)w[i] : 1.0;
            num += wi * (double)y[i];
            den += wi;
        });
    }
    double a = 0, b = 0;
    for (int64_t k = 0; k < nblocks; ++k) { a += s1[(size_t)k]; b += s2[(size_t)k]; }
    return base_from_sums(p, a, b);
}

static std::string effective_metric(const Params &p) {
    if (p.metric != "auto") return p.metric;
    switch (p.objective) {
    case OBJ_MAE: return "mae";
    case OBJ_QUANTILE: return "pinball";
    case OBJ_LOGISTIC: return "logloss";
    case OBJ_POISSON: return "poisson";
    case OBJ_TWEEDIE: return "tweedie";
    case OBJ_MULTICLASS: return "multi_logloss";
    default: return "rmse";
    }
}

// evalMetricRaw (Booster.swift:1855-1918).
static float eval_metric(const Params &p, const float *pred, const float *y, int64_t n) {
    const std::string m = effective_metric(p);
    if (m == "rmse" || m == "auto") {
        double s = 0;
        for (int64_t i = 0; i < n; ++i) { double d = (double)pred[i] - y[i]; s += d * d; }
        return (float)std::sqrt(s / (double)n);
    }
    if (m == "mae") {
        double s = 0;
        for (int64_t i = 0; i < n; ++i) s += std::fabs((double)pred[i] - y[i]);
        return (float)(s / (double)n);
    }
    if (m == "pinball") {
        double a = p.alpha, s = 0;
        for (int64_t i = 0; i < n; ++i) { double d = (double)y[i] - pred[i]; s += d >= 0 ? a * d : (a - 1) * d; }
        return (float)(s / (double)n);
    }
    if (m == "logloss") {
        double s = 0;
        for (int64_t i = 0; i < n; ++i) {
            double q = 1 / (1 + std::exp(-(double)pred[i])), yy = y[i];
            s += -(yy * std::log(std::max(q, 1e-12)) + (1 - yy) * std::log(std::max(1 - q, 1e-12)));
        }
        return (float)(s / (double)n);
    }
    if (m == "auc") {
        std::vector<int64_t> idx((size_t)n);
        for (int64_t i = 0; i < n; ++i) idx[(size_t)i] = i;
        std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) { return pred[a] < pred[b]; });
        double pos_rank = 0, npos = 0;
        int64_t i = 0;
        while (i < n) {
            int64_t j = i;
            while (j < n && pred[idx[(size_t)j]] == pred[idx[(size_t)i]]) ++j;
            double avg = (double)(i + j + 1) / 2;
            for (int64_t k = i; k < j; ++k)
                if (y[idx[(size_t)k]] > 0.5f) { pos_rank += avg; npos += 1; }
            i = j;
        }
        double nneg = (double)n - npos;
        if (!(npos > 0 && nneg > 0)) return 0.5f;
        return (float)((pos_rank - npos * (npos + 1) / 2) / (npos * nneg));
    }
    if (m == "poisson") {
        double s = 0;
        for (int64_t i = 0; i < n; ++i) {
            double mu = std::exp((double)pred[i]), yy = y[i];
            s += 2 * ((yy > 0 ? yy * std::log(yy / mu) : 0) - (yy - mu));
        }
        return (float)(s / (double)n);
    }
    if (m == "tweedie") {
        double rho = p.tweedie_power, s = 0;
        for (int64_t i = 0; i < n; ++i) {
            double mu = std::exp((double)pred[i]), yy = y[i];
            double a = yy > 0 ? std::pow(yy, 2 - rho) / ((1 - rho) * (2 - rho)) : 0;
            s += 2 * (a - yy * std::pow(mu, 1 - rho) / (1 - rho) + std::pow(mu, 2 - rho) / (2 - rho));
        }
        return (float)(s / (double)n);
    }
    return 0.0f;
}

// Checks shared by both entry points (Booster.swift:451-529).
// The per-row checks of validate_inputs: labels, weights, validation labels.
static void validate_rows(const Params &p, int64_t rows, const float *y, const float *w,
                          const float *xv, int64_t vrows, const float *yv) {
    validate_labels(p, y, rows);
    if (w) {
        const int64_t block = 1 << 18;
        std::vector<int64_t> first((size_t)((rows + block - 1) / block), -1);
        parallel_blocks(rows, block, [&](int64_t a, int64_t b) {
            for (int64_t i = a; i < b; ++i)
                if (!(std::isfinite(w[i]) && w[i] >= 0)) { first[(size_t)(a / block)] = i; return; }
        });
        for (int64_t i : first)
            if (i >= 0)
                invalid("weight at row " + std::to_string(i) + " is " + swift_float(w[i]) +
                        "; weights must be finite and >= 0");
    }
    if (xv && yv && vrows > 0) validate_labels(p, yv, vrows);
}

// The shape checks of validate_inputs.
static void validate_shape(const Params &p, int64_t rows, int64_t cols) {
    if (p.has_monotone && (int64_t)p.monotone.size() != cols)
        invalid("monotoneConstraints has " + std::to_string(p.monotone.size()) +
                " entries, X has " + std::to_string(cols) + " features");
    if (p.has_allowed) {
        bool ok = !p.allowed.empty();
        for (int f : p.allowed) ok = ok && f >= 0 && f < cols;
        if (!ok) invalid("allowedFeatures must be non-empty indices within 0..<" + std::to_string(cols));
    }
    if (rows > 0xFFFFFFF0LL) invalid("more than 2^32 rows are not supported");
}

// Input checks in the reference's order (Booster.swift:262-330, :1724-1826).
static void validate_inputs(const Params &p, int64_t rows, int64_t cols, const float *y,
                            const float *w, const float *xv, int64_t vrows, const float *yv) {
    validate_rows(p, rows, y, w, xv, vrows, yv);
    validate_shape(p, rows, cols);
}

// Device, shapes and params-derived constants; t.p holds the effective
// params (bin count and categorical layout included).
static void setup_shape(Trainer &t, int64_t rows, int64_t cols) {
    const Params &p = t.p;
    t.dev = acquire_device(0);
    hipStream_t s = t.dev->stream;
    t.rows = rows;
    t.cols = (int)cols;
    t.nb = p.num_bins;
    t.D = p.max_depth;
    t.total_nodes = (1 << (t.D + 1)) - 1;
    t.max_level_nodes = 1 << (t.D - 1);
    t.is_cat_h.assign((size_t)cols, 0);
    for (int f : p.categorical) t.is_cat_h[(size_t)f] = 1;
    t.has_cats = !p.categorical.empty();
    t.mono_h.assign((size_t)cols, 0);
    if (p.has_monotone)
        for (int64_t f = 0; f < cols; ++f) t.mono_h[(size_t)f] = (int8_t)p.monotone[(size_t)f];
    t.mask_base.assign((size_t)cols, 1);
    if (p.has_allowed)
        for (int64_t f = 0; f < cols; ++f) t.mask_base[(size_t)f] = p.allowed.count((int)f) ? 1 : 0;

    // gather-layout tile width: features per row tile.  64 features per tile
    // for wide matrices (four lanes per gathered row, so one load covers a
    // row's tile); narrower matrices use the smallest tile that holds all
    // features.  (32-wide tiles with the last tile folded in cost fewer LDS adds
    // but three L2 requests per row and item: slower on the gathered levels,
    // faster on the streamed root, which uses them; see root_shape.)
    int tile_w = cols > 32 ? 64 : cols > 16 ? 32 : cols > 8 ? 16 : 8;
    if (const char *e = std::getenv("MACBOOST_TILE_W")) tile_w = std::atoi(e);
    if (tile_w != 8 && tile_w != 16 && tile_w != 32 && tile_w != 64) tile_w = 64;
    t.sh.rows = rows;
    t.sh.cols = (int)cols;
    t.sh.num_bins = p.num_bins;
    t.sh.tile_w = tile_w;
    t.sh.num_tiles = (int)((cols + tile_w - 1) / tile_w);
    // gathered levels never fold: the extras' loads cost more L2 requests there
    // than their saved LDS adds gain (10M x 100, level 1: 129 against 92 us
    // with two lanes per row, worse with one)
    mbk::set_hist_tiling(t.sh, false);
    t.sh_root = t.sh;
    t.sp.lambda = p.lambda;
    t.sp.min_child_hess = p.min_child_hess;
    t.sp.min_split_gain = p.min_split_gain;
    t.sp.cat_smooth = p.cat_smooth;
    t.sp.learning_rate = p.learning_rate;
    t.sp.max_depth = p.max_depth;
    t.gp.objective = p.objective;
    t.gp.alpha = p.alpha;
    t.gp.aux = p.objective == OBJ_LOGISTIC ? p.scale_pos_weight
             : p.objective == OBJ_TWEEDIE ? p.tweedie_power : 0.0f;
    t.is_cat.alloc((size_t)cols);
    MB_HIP(hipMemcpyAsync(t.is_cat.ptr, t.is_cat_h.data(), (size_t)cols, hipMemcpyHostToDevice, s));

    // rows-per-bin hint (Booster.swift:730-738)
    if (rows / p.num_bins < 64 && p.num_bins > 64) {
        int suggest = 64;
        while (suggest > 32 && rows / suggest < 64) suggest /= 2;
        t.warnings.push_back(
            "max_bin=" + std::to_string(p.num_bins) + " gives ~" +
            std::to_string(std::max<int64_t>(1, rows / p.num_bins)) + " rows per bin at " +
            std::to_string(rows) + " rows; max_bin=" + std::to_string(suggest) +
            " is typically 2-4x faster here with equal accuracy (histogram cost scales with "
            "bins, resolution does not once bins exceed rows per node)");
    }
}

// Bins a raw feature-major validation set with the training edges (device).
static void bin_valid(Trainer &t, const float *xv, int64_t vrows, const float *edges_dev) {
    hipStream_t s = t.dev->stream;
    t.has_valid = true;
    t.vrows = vrows;
    DevBuf<float> xvd((size_t)vrows * (size_t)t.cols);
    DevBuf<uint8_t> vt((size_t)t.sh.num_tiles * (size_t)vrows * (size_t)t.sh.tile_w);
    t.vbins_fm.alloc((size_t)vrows * (size_t)t.cols);
    MB_HIP(hipMemcpyAsync(xvd.ptr, xv, xvd.bytes(), hipMemcpyHostToDevice, s));
    MB_HIP(mbk::launch_bin_data(s, xvd.ptr, vrows, t.cols, 1, vrows, edges_dev, t.is_cat.ptr,
                                t.nb, t.sh.tile_w, t.sh.num_tiles, vt.ptr, t.vbins_fm.ptr));
    MB_HIP(hipStreamSynchronize(s));
}

// Labels, weights, predictions and the tree-build buffers.
// The root histogram streams every row.  The gather layout holds T * W B per
// row although the features fill fewer (100 of 128 at F = 100), and the tile
// workgroups of a row chunk read parts of the same lines.  The planar copy
// stores each tile's bytes contiguously (64-wide tiles: the last one at
// ceil(F_last/16)*16 B; 32-wide tiles with extras: the extras in a plane of
// their own), so each workgroup streams its own plane.
// The root's histogram shape: over the planar copy, 32-wide tiles with the
// last tile's features folded in when that applies (F = 100: 34 + 33 + 33 LDS
// adds per 64 rows instead of 128; 223 against 244 us for the 10M-row root),
// else the gather shape.  The copy reads feature f at byte f of a gather row,
// which holds for every tile width.
static mbk::Shape root_shape(const Trainer &t) {
    mbk::Shape r = t.sh;
    r.tile_w = 32;
    r.num_tiles = (t.sh.cols + 31) / 32;
    mbk::set_hist_tiling(r);
    const int32_t row_bytes = t.sh.num_tiles * t.sh.tile_w;
    if (r.extras > 0 && r.hist_tiles * 32 + (r.extras + 3) / 4 * 4 <= row_bytes) return r;
    return t.sh;
}

static void build_root_copy(Trainer &t) {
    t.has_root_copy = false;
    if (!mbk::has_planar_layout(t.sh_root)) return;
    const mbk::HistLayout lay = mbk::planar_layout(t.sh_root);
    hipStream_t s = t.dev->stream;
    const size_t bytes = mbk::planar_bytes(t.sh_root);
    // an optimisation only: skipped unless it leaves 1/16 of the device free
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess || free_b < bytes + (total_b >> 4)) return;
    t.bins_root.alloc(bytes);
    MB_HIP(hipMemsetAsync(t.bins_root.ptr + bytes - 64, 0, 64, s));
    MB_HIP(mbk::launch_planar_rows(s, t.sh_root, t.bins_tiled.ptr,
                                   t.sh.num_tiles * t.sh.tile_w, t.bins_root.ptr));
    t.root_layout = lay;
    t.has_root_copy = true;
}

// Base scores (Booster.swift:786-846): per-class log priors with +1 smoothing
// for multiclass, else one base_score.
static std::vector<float> base_scores_of(const Params &p, const float *y, const float *w,
                                         int64_t rows) {
    if (p.objective == OBJ_MULTICLASS) {
        const int K = p.num_classes;
        std::vector<double> cnt((size_t)K, 1.0);
        for (int64_t i = 0; i < rows; ++i) cnt[(size_t)y[i]] += w ? (double)w[i] : 1.0;
        double total = 0;
        for (double c : cnt) total += c;
        std::vector<float> out((size_t)K);
        for (int k = 0; k < K; ++k) out[(size_t)k] = (float)std::log(cnt[(size_t)k] / total);
        return out;
    }
    Phase ph("base score");
    return {base_score(p, y, w, rows)};
}

static void setup_buffers(Trainer &t, const float *y, const float *w, const float *yv,
                          const std::vector<float> *bases = nullptr) {
    const Params &p = t.p;
    hipStream_t s = t.dev->stream;
    const int64_t rows = t.rows, cols = t.cols, vrows = t.vrows;
    t.gp.has_weights = w ? 1 : 0;
    // --- persistent buffers ---------------------------------------------
    t.K = p.objective == OBJ_MULTICLASS ? p.num_classes : 1;
    const int K = t.K;
    t.gp.num_classes = K;
    t.gp.class_index = 0;
    t.gp.rows = rows;
    // the host keeps no copy of the labels: a train metric reads them back
    if (!t.labels_ready) {
        t.labels.alloc((size_t)rows);
        upload(t.labels.ptr, y, (size_t)rows * 4, s);
    }
    t.preds.alloc((size_t)rows * (size_t)K);
    if (w) {
        t.has_weights = true;
        if (!t.weights_ready) {
            t.weights.alloc((size_t)rows);
            upload(t.weights.ptr, w, (size_t)rows * 4, s);
        }
    }
    t.base_scores = bases ? *bases : base_scores_of(p, y, w, rows);
    t.base = K > 1 ? 0.0f : t.base_scores[0];
    if (t.has_valid) {
        t.vlabels_h.assign(yv, yv + vrows);
        t.vpreds.alloc((size_t)vrows * (size_t)K);
    }
    for (int k = 0; k < K; ++k) {
        uint32_t bits;
        std::memcpy(&bits, &t.base_scores[(size_t)k], 4);
        MB_HIP(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(t.preds.ptr + (size_t)k * rows),
                                 (int)bits, (size_t)rows, s));
        if (t.has_valid)
            MB_HIP(hipMemsetD32Async(
                reinterpret_cast<hipDeviceptr_t>(t.vpreds.ptr + (size_t)k * vrows), (int)bits,
                (size_t)vrows, s));
    }
    if (!t.seed_train.empty()) {
        // warm start: preds [K][rows] from the init model's raw scores [rows][K]
        std::vector<float> cm((size_t)rows * (size_t)K);
        for (int64_t i = 0; i < rows; ++i)
            for (int k = 0; k < K; ++k)
                cm[(size_t)k * rows + i] = t.seed_train[(size_t)(i * K + k)];
        MB_HIP(hipMemcpyAsync(t.preds.ptr, cm.data(), cm.size() * 4, hipMemcpyHostToDevice, s));
        MB_HIP(hipStreamSynchronize(s));
        if (t.has_valid && !t.seed_valid.empty()) {
            std::vector<float> vm((size_t)vrows * (size_t)K);
            for (int64_t i = 0; i < vrows; ++i)
                for (int k = 0; k < K; ++k)
                    vm[(size_t)k * vrows + i] = t.seed_valid[(size_t)(i * K + k)];
            MB_HIP(hipMemcpyAsync(t.vpreds.ptr, vm.data(), vm.size() * 4, hipMemcpyHostToDevice, s));
            MB_HIP(hipStreamSynchronize(s));
        }
        t.seed_train.clear();
        t.seed_train.shrink_to_fit();
        t.seed_valid.clear();
        t.seed_valid.shrink_to_fit();
    }
    t.preds_cur = t.preds.ptr;
    t.vpreds_cur = t.has_valid ? t.vpreds.ptr : nullptr;
    t.mono.alloc((size_t)cols);
    MB_HIP(hipMemcpyAsync(t.mono.ptr, t.mono_h.data(), (size_t)cols, hipMemcpyHostToDevice, s));
    t.feat_mask.alloc((size_t)cols);
    MB_HIP(hipMemcpyAsync(t.feat_mask.ptr, t.mask_base.data(), (size_t)cols, hipMemcpyHostToDevice, s));

    t.leafwise = p.num_leaves > 0;
    if (t.leafwise) {
        t.order_a.alloc((size_t)rows * 2);           // both halves of the partition buffer
    } else {
        t.order_a.alloc((size_t)rows);
        t.order_b.alloc((size_t)rows);
    }
    t.gmax_part.alloc(mbk::grad_max_scratch_words());
    if (p.goss || p.subsample < 1.0f) {
        t.samp_g.alloc((size_t)rows);
        t.samp_h.alloc((size_t)rows);
        t.samp_h_kept.alloc((size_t)rows);
        t.goss_buckets.alloc(1024);
        MB_HIP(hipMemsetAsync(t.goss_buckets.ptr, 0, 1024 * sizeof(uint32_t), s));
    }
    // level-wise partition: one block per PART_ENTRIES entries of a split node
    // persistent partition grid: two 1024-thread blocks per CU, or fewer when
    // a level can never need that many
    t.route_grid = (uint32_t)std::min<int64_t>(
        2 * (int64_t)t.dev->num_cus,
        (rows + mbk::PART_ENTRIES - 1) / mbk::PART_ENTRIES + t.max_level_nodes);
    t.route_cursor.alloc((size_t)t.max_level_nodes * mbk::CURSOR_STRIDE);
    t.split_keys.alloc((size_t)t.max_level_nodes * mbk::SPLIT_KEY_STRIDE);
    t.route_done.alloc(1);
    MB_HIP(hipMemsetAsync(t.route_done.ptr, 0, sizeof(uint32_t), t.dev->stream));

    // histogram work decomposition: one workgroup per CU (128 KiB of LDS),
    // one item per workgroup and round
    t.hist_grid = t.dev->num_cus;
    t.target_items = t.hist_grid;
    t.min_chunk = 2048;
    // a level's items: T*ceil(count/chunk) summed over its built nodes, at most
    // target*rounds + T*nodes, where target*rounds <= T*rows/HIST_CHUNK_MAX + target
    auto max_items_of = [&](int64_t T, int64_t nodes, int64_t target) {
        const int64_t m = T * ((rows + mbk::HIST_CHUNK_MAX - 1) / mbk::HIST_CHUNK_MAX) +
                          target + 1 + T * nodes;
        return std::min<int64_t>(m, T * ((rows + t.min_chunk - 1) / t.min_chunk + nodes + 1));
    };
    t.sh_root = root_shape(t);
    t.sh.item_cap = (uint32_t)max_items_of(t.sh.hist_tiles, t.max_level_nodes, t.target_items);
    t.sh_root.item_cap = (uint32_t)max_items_of(t.sh_root.hist_tiles, t.max_level_nodes,
                                                t.target_items);
    t.partials.alloc(std::max((size_t)t.sh.item_cap * (size_t)t.sh.part_w,
                              (size_t)t.sh_root.item_cap * (size_t)t.sh_root.part_w) *
                     (size_t)p.num_bins);
    t.items.alloc((size_t)std::max(t.sh.item_cap, t.sh_root.item_cap));
    t.pairs.alloc((size_t)t.max_level_nodes);
    // Leaf-wise trees up to depth LWB_MAX_DEPTH grow in depth rounds on the
    // level-wise buffers, unless two levels of histograms would pass 4 GiB
    const size_t level_hist_bytes =
        (size_t)t.max_level_nodes * cols * p.num_bins * 2 * sizeof(int64_t);
    t.lw_rounds = t.leafwise && t.D <= mbk::LWB_MAX_DEPTH &&
                  p.num_leaves <= mbk::LWB_MAX_LEAVES && 2 * level_hist_bytes <= ((size_t)4 << 30);
    // level-wise (and leaf-wise rounds): two levels of max_level_nodes
    // histograms; leaf-wise steps: one slot per evaluated leaf (at most num_leaves)
    const bool level_bufs = !t.leafwise || t.lw_rounds;
    const size_t slots = level_bufs ? (size_t)t.max_level_nodes : (size_t)p.num_leaves;
    const size_t hist_n = slots * cols * p.num_bins * 2;
    t.hist_a.alloc(hist_n);
    if (level_bufs) t.hist_b.alloc(hist_n);
    if (t.lw_rounds) {
        t.lwb.num_leaves = p.num_leaves;
        t.lwb.max_depth = t.D;
        t.lwb.total_nodes = t.total_nodes;
        t.lwb_state.alloc(1);
        t.lwb_cand.alloc((size_t)t.total_nodes);
        t.spec_split.alloc((size_t)t.total_nodes);
        t.spec_cover.alloc((size_t)t.total_nodes);
        t.spec_mask.alloc((size_t)t.total_nodes * 8);
    }
    t.results.alloc(std::max(slots, (size_t)t.max_level_nodes) * cols);
    if (t.leafwise) {
        t.lw.num_leaves = p.num_leaves;
        t.lw.max_depth = t.D;
        t.lw.rows = (uint32_t)rows;
        t.lw.part_blocks = (uint32_t)std::min<int64_t>(
            2 * t.dev->num_cus, (rows + mbk::PART_ENTRIES - 1) / mbk::PART_ENTRIES);
        t.lw.total_nodes = t.total_nodes;
        t.lw.target_items = (uint32_t)t.target_items;
        t.lw.min_chunk = (uint32_t)t.min_chunk;
        t.lw_state.alloc(1);
        t.lw_open.alloc((size_t)2 * p.num_leaves + 2);
    }
    t.renewal = p.objective == OBJ_MAE || p.objective == OBJ_QUANTILE;
    // A sampled level-wise tree counts its deepest nodes' kept rows in the
    // terminal walk.  With min_child_hess > 0 every split child holds a kept
    // row (both sides of a chosen split have hessian >= min_child_hess), so
    // no leaf the walk applies is later emptied and zeroed.
    t.kept_walk = !t.leafwise && (p.goss || p.subsample < 1.0f) && p.min_child_hess > 0.0f &&
                  !t.renewal;
    if (t.kept_walk) t.kept.alloc((size_t)rows);
    if (t.renewal) {
        t.renewal_q = p.objective == OBJ_MAE ? 0.5f : p.alpha;
        const size_t ns = mbk::renew_sample_count(rows);
        t.rn_leaf.alloc(ns);
        t.rn_keys.alloc(ns);
        t.rn_seg.alloc(ns);
        t.rn_cnt.alloc((size_t)t.total_nodes);
        t.rn_off.alloc((size_t)t.total_nodes);
        t.rn_cursor.alloc((size_t)t.total_nodes);
        t.rn_delta.alloc((size_t)t.total_nodes);
    }
    t.count.alloc((size_t)t.total_nodes);
    t.node_g.alloc((size_t)t.total_nodes);
    t.node_h.alloc((size_t)t.total_nodes);
    t.bounds.alloc((size_t)t.total_nodes);
    t.seg_a.alloc((size_t)1 << t.D);
    t.seg_b.alloc((size_t)1 << t.D);
    t.ctl.alloc(1);
    t.ensure_capacity(std::max(1, p.num_trees));
    if (!t.has_root_copy) build_root_copy(t);   // (create_raw builds it after the binning)
    MB_HIP(hipStreamSynchronize(s));
    t.best_metric = effective_metric(p) == "auc" ? -INFINITY : INFINITY;
}

// Leakage and categorical checks of device-resident features: the leakage
// check reads a strided row sample copied to the host, and the categorical
// ids are checked on the device (the first offending row of the first
// offending feature gives the host path's message).
// Device features: the categorical id rule is checked on the device; the
// rows the leakage check samples (every max(1, rows/4096)-th) are copied to
// xs [m][cols] with their labels in ys, for check_leakage on the host
// (every row of that sample is used: its step is 1, m < 8192).
static void check_device_features(const Params &p, const float *x_dev, int64_t rows,
                                  int64_t cols, int64_t rs, int64_t cs, const float *y,
                                  hipStream_t s, std::vector<float> &xs, std::vector<float> &ys) {
    const int64_t step = std::max<int64_t>(1, rows / 4096);
    const int64_t m = (rows + step - 1) / step;
    xs.clear();
    ys.clear();
    if (m >= 50) {
        DevBuf<float> sd;                               // released after the stream drained
        sd.pooled = true;
        sd.alloc((size_t)(m * cols));
        xs.resize((size_t)(m * cols));
        ys.resize((size_t)m);
        MB_HIP(mbk::launch_gather_sample(s, x_dev, rs, cs, step, m, (int)cols, sd.ptr));
        MB_HIP(hipMemcpyAsync(xs.data(), sd.ptr, sd.bytes(), hipMemcpyDeviceToHost, s));
        MB_HIP(hipStreamSynchronize(s));
        for (int64_t k = 0; k < m; ++k) ys[(size_t)k] = y[k * step];
    }
    if (p.categorical.empty()) return;
    std::vector<int32_t> cat(p.categorical.begin(), p.categorical.end());
    for (int f : cat)
        if (f < 0 || f >= cols)
            internal("categorical feature index " + std::to_string(f) + " out of range");
    DevBuf<int32_t> cd(cat.size());
    DevBuf<uint32_t> bad(cat.size());
    std::vector<uint32_t> first(cat.size());
    MB_HIP(hipMemcpyAsync(cd.ptr, cat.data(), cd.bytes(), hipMemcpyHostToDevice, s));
    MB_HIP(hipMemsetAsync(bad.ptr, 0xFF, bad.bytes(), s));
    MB_HIP(mbk::launch_check_categorical(s, x_dev, rows, rs, cs, cd.ptr, (int)cat.size(),
                                         p.num_bins - 1, bad.ptr));
    MB_HIP(hipMemcpyAsync(first.data(), bad.ptr, bad.bytes(), hipMemcpyDeviceToHost, s));
    MB_HIP(hipStreamSynchronize(s));
    for (size_t j = 0; j < cat.size(); ++j) {
        if (first[j] == 0xFFFFFFFFu) continue;
        float v = 0;
        MB_HIP(hipMemcpy(&v, x_dev + (int64_t)first[j] * rs + (int64_t)cat[j] * cs, 4,
                         hipMemcpyDeviceToHost));
        throw Error("Categorical feature " + std::to_string(cat[j]) + " has value " +
                    swift_float(v) + "; expected integer ids in 0..<" +
                    std::to_string(p.num_bins - 1) + " or NaN");
    }
}

// fitImpl's setup (Booster.swift:445-600) for raw features in host memory
// (x_on_device false: uploaded here) or already in device memory.
static Trainer *create_raw(const Params &pin, const float *x, bool x_on_device, int64_t rows,
                           int64_t cols, bool row_major, const float *y, const float *w,
                           const float *xv, int64_t vrows, const float *yv) {
    if (!x || !y || rows <= 0 || cols <= 0) internal("null or empty training data");
    Phase ph_all("fit setup");
    validate_params(pin);
    // The per-row checks (labels, weights) and the base scores: for objectives
    // whose base score sums every row, on the device right after the labels
    // arrive (k_label_stats); for the others on a host thread while the
    // device is set up and the features binned.  The checks keep the
    // reference's order: a later check's error is reported only when the row
    // checks pass.
    const bool dev_rows = sums_base(pin);
    struct HostPrep {
        std::thread th;
        std::exception_ptr err;
        std::vector<float> bases;
        void join() { if (th.joinable()) th.join(); }
        ~HostPrep() { join(); }
    } prep;
    if (!dev_rows) {
        prep.th = std::thread([&] {
            try {
                Phase ph("validate inputs");
                validate_rows(pin, rows, y, w, xv, vrows, yv);
                prep.bases = base_scores_of(pin, y, w, rows);
            } catch (...) {
                prep.err = std::current_exception();
            }
        });
    }
    try {
        validate_shape(pin, rows, cols);
        auto tr = std::make_unique<Trainer>();
        Trainer &t = *tr;
        t.p = pin;
        t.user_params = pin;
        const Params &p = t.p;
        const int64_t rs = row_major ? cols : 1, cs = row_major ? 1 : rows;
        std::unique_ptr<Booster> im;
        if (!p.init_model.empty()) {                     // Booster.swift:487-499
            if (x_on_device) invalid("initModel needs the raw features in host memory");
            im.reset(load_model_file(p.init_model));
            if (im->num_features != cols)
                invalid("initModel expects " + std::to_string(im->num_features) + " features, X has " +
                        std::to_string(cols));
            if (im->params.objective != p.objective) invalid("initModel objective differs");
            const int k_want = p.objective == OBJ_MULTICLASS ? p.num_classes : 1;
            if (std::max(1, im->trained_num_classes) != k_want)
                invalid("initModel has " + std::to_string(im->trained_num_classes) +
                        " classes, the params ask for " + std::to_string(k_want));
        }
        // host features: the leakage check runs on a host thread while the device
        // is set up and the data uploaded and binned (a failure there is rethrown
        // on this thread after the join)
        std::vector<std::string> leak_warnings;
        std::exception_ptr leak_error;
        std::vector<float> leak_xs, leak_ys;         // device features: the sampled rows
        struct Joiner {
            std::thread th;
            ~Joiner() { if (th.joinable()) th.join(); }
        } leak;
        if (!x_on_device) {
            leak.th = std::thread([&] {
                try {
                    check_leakage(p.verbose, x, rows, cols, rs, cs, y, leak_warnings);
                } catch (...) {
                    leak_error = std::current_exception();
                }
            });
            validate_categoricals(p, x, rows, cols, rs, cs);
        }
        if (xv && yv && vrows > 0) validate_categoricals(p, xv, vrows, cols, 1, vrows);
        setup_shape(t, rows, cols);
        hipStream_t s = t.dev->stream;
        const int tile_w = t.sh.tile_w;
        if (x_on_device) {
            Phase ph("device feature checks");
            check_device_features(p, x, rows, cols, rs, cs, y, s, leak_xs, leak_ys);
            if (!leak_ys.empty()) {
                leak.th = std::thread([&] {
                    try {
                        check_leakage(p.verbose, leak_xs.data(), (int64_t)leak_ys.size(), cols,
                                      cols, 1, leak_ys.data(), leak_warnings);
                    } catch (...) {
                        leak_error = std::current_exception();
                    }
                });
            }
        }

        // --- binning on the device: (upload,) quantile edges, bin_data --------
        std::vector<mbk::LabelStats> row_stats;       // the device row checks' blocks
        double t0 = now_s(), te = t0;
        struct Events {                              // destroyed after the streams drained
            std::vector<hipEvent_t> ev;
            ~Events() { for (hipEvent_t e : ev) (void)hipEventDestroy(e); }
        } tile_ready;
        {
            DevBuf<float> xd;                           // host features: kept in the cache
            xd.pooled = true;                           // (no 4 GB hipMalloc / hipFree per fit)
            const float *xsrc = x;
            if (!x_on_device) {
                xd.alloc((size_t)rows * (size_t)cols);
                xsrc = xd.ptr;
            }
            const size_t ne = (size_t)p.num_bins - 2;
            DevBuf<float> ed;                           // released after the stream drained
            ed.pooled = true;
            ed.alloc(std::max<size_t>(1, (size_t)cols * ne));
            const size_t cap = mbk::edge_sample_cap(rows);
            DevBuf<uint32_t> ka, kb, cnt;               // released after the stream drained
            ka.pooled = kb.pooled = cnt.pooled = true;
            ka.alloc((size_t)cols * cap);
            kb.alloc((size_t)cols * cap);
            cnt.alloc((size_t)cols);
            t.bins_tiled.alloc((size_t)t.sh.num_tiles * (size_t)rows * (size_t)tile_w);
            t.bins_fm.alloc((size_t)rows * (size_t)cols);
            const int T = t.sh.num_tiles;
            if (!x_on_device && !row_major && T > 1) {
                // Feature-major host features arrive one tile's columns at a
                // time on the copy stream; each tile's quantile edges and
                // binning run on the compute stream while the next tile's
                // columns cross PCIe, so only the last tile's work follows the
                // upload (FitTimings' prep + bin, Booster.swift:564-566, with
                // the copy overlapped).
                Phase ph("upload + edges + bin data, by tile");
                hipStream_t cps = t.dev->copy_stream;
                for (int tt = 0; tt < T; ++tt) {
                    const int64_t c0 = (int64_t)tt * tile_w;
                    const int64_t nc = std::min<int64_t>(tile_w, cols - c0);
                    upload(xd.ptr + c0 * rows, x + c0 * rows, (size_t)(nc * rows) * sizeof(float),
                           cps);
                    hipEvent_t ev = nullptr;
                    MB_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
                    tile_ready.ev.push_back(ev);
                    MB_HIP(hipEventRecord(ev, cps));
                    MB_HIP(hipStreamWaitEvent(s, ev, 0));
                    MB_HIP(mbk::launch_edges(s, xd.ptr + c0 * rows, rows, (int)nc, 1, rows,
                                             p.num_bins, t.is_cat.ptr + c0, ka.ptr, kb.ptr, cnt.ptr,
                                             ed.ptr + c0 * (int64_t)ne));
                    MB_HIP(mbk::launch_bin_tiles(s, xd.ptr, rows, (int)cols, 1, rows, ed.ptr,
                                                 t.is_cat.ptr, p.num_bins, tile_w, T, tt, 1,
                                                 t.bins_tiled.ptr, t.bins_fm.ptr));
                }
                te = now_s();
            } else {
                if (!x_on_device) upload(xd.ptr, x, xd.bytes(), s);
                te = now_s();
                {
                    Phase ph("quantile edges");
                    MB_HIP(mbk::launch_edges(s, xsrc, rows, (int)cols, rs, cs, p.num_bins,
                                             t.is_cat.ptr, ka.ptr, kb.ptr, cnt.ptr, ed.ptr));
                }
                // binning follows the edges on the device; meanwhile the labels
                // cross PCIe on the copy stream and the edges come back to the host
                Phase ph("bin data");
                MB_HIP(mbk::launch_bin_data(s, xsrc, rows, (int)cols, rs, cs, ed.ptr, t.is_cat.ptr,
                                            p.num_bins, tile_w, t.sh.num_tiles, t.bins_tiled.ptr,
                                            t.bins_fm.ptr));
            }
            // the root pass's planar copy follows the binning on the compute
            // stream, and the labels cross PCIe and are checked meanwhile; the
            // edges' copy to the host waits for both kernels
            t.sh_root = root_shape(t);
            build_root_copy(t);
            hipStream_t cs2 = t.dev->copy_stream;
            t.labels.alloc((size_t)rows);
            upload(t.labels.ptr, y, (size_t)rows * 4, cs2);
            t.labels_ready = true;
            if (dev_rows) {
                // the row checks and the base score's sums, on the device
                if (w) {
                    t.weights.alloc((size_t)rows);
                    upload(t.weights.ptr, w, (size_t)rows * 4, cs2);
                    t.weights_ready = true;
                }
                const size_t nblk = mbk::label_stats_blocks(rows);
                DevBuf<mbk::LabelStats> ls;
                ls.pooled = true;
                ls.alloc(nblk);
                MB_HIP(mbk::launch_label_stats(cs2, p.objective, p.num_classes, t.labels.ptr,
                                               w ? t.weights.ptr : nullptr, rows,
                                               p.scale_pos_weight, ls.ptr));
                row_stats.resize(nblk);
                MB_HIP(hipMemcpyAsync(row_stats.data(), ls.ptr, nblk * sizeof(mbk::LabelStats),
                                      hipMemcpyDeviceToHost, cs2));
                MB_HIP(hipStreamSynchronize(cs2));
            }
            t.edges.resize((size_t)cols * ne);
            MB_HIP(hipMemcpyAsync(t.edges.data(), ed.ptr, t.edges.size() * 4, hipMemcpyDeviceToHost, s));
            MB_HIP(hipStreamSynchronize(cs2));
            if (xv && yv && vrows > 0) bin_valid(t, xv, vrows, ed.ptr);
            MB_HIP(hipStreamSynchronize(s));
            t.t_edges = now_s() - te;
        }
        t.t_bin = now_s() - t0 - t.t_edges;              // the feature upload, if any
        prep.join();
        if (prep.err) std::rethrow_exception(prep.err);
        if (dev_rows) {
            // labels, then weights, then the validation labels (validate_rows)
            int64_t bad_y = INT64_MAX, bad_w = INT64_MAX;
            double s1 = 0, s2 = 0;
            for (const mbk::LabelStats &b : row_stats) {
                bad_y = std::min(bad_y, b.bad_label);
                bad_w = std::min(bad_w, b.bad_weight);
                s1 += b.s1;
                s2 += b.s2;
            }
            if (bad_y != INT64_MAX) check_label(p, y, bad_y);
            if (bad_w != INT64_MAX)
                invalid("weight at row " + std::to_string(bad_w) + " is " + swift_float(w[bad_w]) +
                        "; weights must be finite and >= 0");
            if (xv && yv && vrows > 0) validate_labels(p, yv, vrows);
            prep.bases = {base_from_sums(p, s1, s2)};
        }
        Phase ph_rest("labels, buffers");
        if (leak.th.joinable()) leak.th.join();
        if (leak_error) std::rethrow_exception(leak_error);
        t.warnings.insert(t.warnings.begin(), leak_warnings.begin(), leak_warnings.end());
        if (im) {
            // the init model's raw scores on the training (and validation) rows
            if (row_major) {
                std::vector<float> xfm((size_t)rows * (size_t)cols);
                for (int64_t i = 0; i < rows; ++i)
                    for (int64_t f = 0; f < cols; ++f) xfm[(size_t)(f * rows + i)] = x[i * cols + f];
                t.seed_train = im->predict_raw(xfm.data(), rows, cols);
            } else {
                t.seed_train = im->predict_raw(x, rows, cols);
            }
            if (xv && yv && vrows > 0) t.seed_valid = im->predict_raw(xv, vrows, cols);
            t.init_trees = im->trees;
        }
        setup_buffers(t, y, w, yv, &prep.bases);
        if (im) {
            t.base = im->base_score;
            t.base_scores = im->base_scores;
        }
        return tr.release();
    } catch (...) {
        // the row checks come first in the reference's order
        prep.join();
        if (prep.err) std::rethrow_exception(prep.err);
        if (dev_rows) validate_rows(pin, rows, y, w, xv, vrows, yv);
        throw;
    }
}

Trainer *trainer_create(const Params &p, const float *x, int64_t rows, int64_t cols,
                        bool row_major, const float *y, const float *w, const float *xv,
                        int64_t vrows, const float *yv) {
    return create_raw(p, x, false, rows, cols, row_major, y, w, xv, vrows, yv);
}

Trainer *trainer_create_device(const Params &p, const float *x_dev, int64_t rows, int64_t cols,
                               bool row_major, const float *y, const float *w, const float *xv,
                               int64_t vrows, const float *yv) {
    return create_raw(p, x_dev, true, rows, cols, row_major, y, w, xv, vrows, yv);
}

// fitImpl with GPU-resident pre-binned input (GPUBinned, Booster.swift:436-443,
// feature selection's shadow matrix): feature-major device bins [cols][rows],
// rearranged into the gather layout on the device.
Trainer *trainer_create_fm(const Params &pin, int64_t rows, int64_t cols, const uint8_t *fm_dev,
                           const std::vector<float> &edges, const float *y, const float *w) {
    validate_params(pin);
    validate_inputs(pin, rows, cols, y, w, nullptr, 0, nullptr);
    auto tr = std::make_unique<Trainer>();
    Trainer &t = *tr;
    t.p = pin;
    t.user_params = pin;
    setup_shape(t, rows, cols);
    hipStream_t s = t.dev->stream;
    {
        const int64_t groups = (cols + 7) / 8;
        DevBuf<uint64_t> words((size_t)groups * (size_t)rows);
        DevBuf<uint32_t> bad(1);
        MB_HIP(hipMemsetAsync(bad.ptr, 0, 4, s));
        t.bins_tiled.alloc((size_t)t.sh.num_tiles * (size_t)rows * (size_t)t.sh.tile_w);
        t.bins_fm.alloc((size_t)rows * (size_t)cols);
        MB_HIP(hipMemsetAsync(t.bins_tiled.ptr, 0, t.bins_tiled.bytes(), s));
        MB_HIP(mbk::launch_fm_to_tile8(s, fm_dev, rows, (int)cols, words.ptr));
        MB_HIP(mbk::launch_tile8_to_layouts(s, words.ptr, rows, (int)cols, t.nb, t.sh.tile_w,
                                            t.sh.num_tiles, t.bins_tiled.ptr, t.bins_fm.ptr,
                                            bad.ptr));
        MB_HIP(hipStreamSynchronize(s));
    }
    t.edges = edges;
    setup_buffers(t, y, w, nullptr);
    return tr.release();
}

// fit(dataset:) (Booster.swift:375-389): the dataset's bin count,
// categorical layout, edges and labels are used; binning is skipped and the
// tile-8 bins are rearranged into the device layouts.
Trainer *trainer_create_binned(const Params &pin, const BinnedDataset &ds, const float *w,
                               const float *xv, int64_t vrows, const float *yv) {
    const int64_t rows = ds.rows, cols = ds.cols;
    if (rows <= 0 || cols <= 0) invalid("training data is empty (rows=" + std::to_string(rows) +
                                        ", cols=" + std::to_string(cols) + ")");
    validate_params(pin);
    Params pe = pin;
    pe.num_bins = ds.num_bins;
    pe.categorical = std::set<int>(ds.categorical.begin(), ds.categorical.end());
    validate_params(pe);
    validate_inputs(pe, rows, cols, ds.labels.data(), w, xv, vrows, yv);
    if (!pin.init_model.empty())                     // Booster.swift:487-491
        invalid("initModel requires raw features (not a prebinned dataset)");
    auto tr = std::make_unique<Trainer>();
    Trainer &t = *tr;
    t.p = pe;
    t.user_params = pin;
    t.has_feature_names = ds.has_feature_names;
    t.feature_names = ds.feature_names;
    if (xv && yv && vrows > 0) validate_categoricals(pe, xv, vrows, cols, 1, vrows);
    setup_shape(t, rows, cols);
    hipStream_t s = t.dev->stream;
    double t0 = now_s();
    {
        const int64_t groups = (cols + 7) / 8;
        DevBuf<uint64_t> in((size_t)groups * (size_t)rows);
        DevBuf<uint32_t> bad(1);
        MB_HIP(hipMemcpyAsync(in.ptr, ds.bins.data(), in.bytes(), hipMemcpyHostToDevice, s));
        MB_HIP(hipMemsetAsync(bad.ptr, 0, 4, s));
        t.bins_tiled.alloc((size_t)t.sh.num_tiles * (size_t)rows * (size_t)t.sh.tile_w);
        t.bins_fm.alloc((size_t)rows * (size_t)cols);
        MB_HIP(hipMemsetAsync(t.bins_tiled.ptr, 0, t.bins_tiled.bytes(), s));
        MB_HIP(mbk::launch_tile8_to_layouts(s, in.ptr, rows, (int)cols, t.nb, t.sh.tile_w,
                                            t.sh.num_tiles, t.bins_tiled.ptr, t.bins_fm.ptr,
                                            bad.ptr));
        uint32_t nbad = 0;
        MB_HIP(hipMemcpyAsync(&nbad, bad.ptr, 4, hipMemcpyDeviceToHost, s));
        MB_HIP(hipStreamSynchronize(s));
        if (nbad) invalid(".mbds bins hold values >= numBins");
        t.edges = ds.edges;
        if (xv && yv && vrows > 0) {
            DevBuf<float> ed(std::max<size_t>(1, t.edges.size()));
            if (!t.edges.empty())
                MB_HIP(hipMemcpyAsync(ed.ptr, t.edges.data(), t.edges.size() * 4,
                                      hipMemcpyHostToDevice, s));
            bin_valid(t, xv, vrows, ed.ptr);
        }
    }
    t.t_bin = now_s() - t0;
    setup_buffers(t, ds.labels.data(), w, yv);
    return tr.release();
}

// Per-tree column sample (Booster.swift:1386-1400).
static const uint8_t *tree_feature_mask(Trainer &t, int tree) {
    if (!(t.p.feature_fraction < 1.0f)) return nullptr;
    std::vector<uint8_t> m((size_t)t.cols, 0);
    uint64_t s = 0xC0150001ULL + (uint64_t)tree * 0x9E3779B97F4A7C15ULL;
    auto next = [&]() {
        s += 0x9E3779B97F4A7C15ULL;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    };
    bool any = false;
    for (int f = 0; f < t.cols; ++f) {
        bool keep = t.mask_base[(size_t)f] == 1 &&
                    (float)(next() >> 40) * (1.0f / 16777216.0f) < t.p.feature_fraction;
        m[(size_t)f] = keep ? 1 : 0;
        any = any || keep;
    }
    if (!any) {
        std::vector<int> cand;
        for (int f = 0; f < t.cols; ++f)
            if (t.mask_base[(size_t)f] == 1) cand.push_back(f);
        m[(size_t)cand[(size_t)(next() % cand.size())]] = 1;
    }
    t.tree_masks.push_back(std::move(m));
    return t.tree_masks.back().data();
}

// Leaf renewal of a finished tree (L1 / quantile objectives): residual
// quantiles of the sampled rows replace its leaf values; with delta, the
// change of each leaf is recorded for preds that already hold the old values.
static void renew_tree(Trainer &t, const mbk::TreeOut &out, float *delta) {
    MB_HIP(mbk::launch_renew(t.dev->stream, t.bins_fm.ptr, t.rows, t.nb, t.D, out,
                             t.labels.ptr, t.preds_cur, t.bounds.ptr, t.renewal_q,
                             t.p.learning_rate, t.rn_leaf.ptr, t.rn_keys.ptr, t.rn_seg.ptr,
                             t.rn_cnt.ptr, t.rn_off.ptr, t.rn_cursor.ptr, delta));
}

// GOSS after ceil(1/learning_rate) warm-up trees, bagging on every tree
// (gossActive / bagging, Booster.swift:1382-1384, :617).
static bool tree_sampled(const Params &p, int tree) {
    if (p.goss) return tree >= (int)std::ceil(1.0f / p.learning_rate);
    return p.subsample < 1.0f;
}

// Keep rates and amplification of a sampled tree (Booster.swift:1401-1434).
static mbk::SampleParams sample_params(const Trainer &t, int tree) {
    const Params &p = t.p;
    mbk::SampleParams s{};
    s.goss = p.goss ? 1 : 0;
    s.top_count = p.goss ? (uint32_t)((float)t.rows * p.goss_top_rate) : 0u;
    s.other_prob = p.goss ? p.goss_other_rate / (1.0f - p.goss_top_rate) : p.subsample;
    s.weight = p.goss ? (1.0f - p.goss_top_rate) / p.goss_other_rate : 1.0f;
    s.seed = (uint32_t)tree + 1u;
    return s;
}

// Gradients, maxima and the tree's order entries: every row quantised, or
// the rows a GOSS / bagging tree keeps (their count stays on the device).
// With root_cover non-null the pass that writes the root's entries also plans
// the root level (its first workgroup, while the others quantise), in place
// of a separate launch_plan_root after it.
static bool tree_entries(Trainer &t, int tree, mbk::TreeCtl *ctl, mbk::Entry *order,
                         uint8_t *kept = nullptr, bool implicit_rows = false,
                         float *root_cover = nullptr) {
    hipStream_t s = t.dev->stream;
    const bool sampled = tree_sampled(t.p, tree);
    mbk::RootPlan rp{};
    if (root_cover) {
        const bool planar = !sampled && t.has_root_copy;
        rp.sh = planar ? t.sh_root : t.sh;
        rp.rows_active = sampled ? mbk::NONE : (uint32_t)t.rows;
        rp.target_items = (uint32_t)t.target_items;
        rp.min_chunk = (uint32_t)t.min_chunk;
        rp.ctl = ctl;
        rp.seg_start = t.seg_a.ptr;
        rp.count = t.count.ptr;
        rp.pairs = t.pairs.ptr;
        rp.items = t.items.ptr;
        rp.cover = root_cover;
        rp.bounds = t.bounds.ptr;
        rp.lo = -INFINITY;
        rp.hi = INFINITY;
    }
    const mbk::RootPlan *plan = root_cover ? &rp : nullptr;
    // the previous tree's deferred fixup: in this root pass's first workgroup
    // when there is one, else on its own
    mbk::PendingFixup fix = t.fix_pending;
    t.fix_pending.active = 0;
    if (fix.active) fix.out = t.tree_out(t.fix_tree);
    if (fix.active && !plan) {
        MB_HIP(mbk::launch_final_fixup(s, fix.la, fix.count, fix.out, fix.zero_empty != 0));
        fix.active = 0;
    }
    const mbk::PendingFixup *fixp = fix.active ? &fix : nullptr;
    // the previous tree's control block goes to ctl_hist, then this tree's
    // starts from zero; when the previous tree's walk computed these
    // gradients (and stored g, h for a sampled tree), only the maxima's final
    // reduction is left, done in the same launch
    mbk::TreeCtl *prev = t.ctl_pending >= 0 ? t.ctl_hist.ptr + t.ctl_pending : nullptr;
    t.ctl_pending = -1;
    // a sampled tree whose gradients the walk computed leaves its start to the
    // sampling's first pass
    const int walk_parts = t.walk_gparts;
    const bool start_in_sample = sampled && walk_parts > 0;
    if (!start_in_sample)
        MB_HIP(mbk::launch_tree_start(s, ctl, prev, walk_parts > 0 ? t.gmax_part.ptr : nullptr,
                                      walk_parts));
    if (t.walk_gparts > 0) {
        t.walk_gparts = 0;
    } else {
        MB_HIP(mbk::launch_grad_max(s, t.gp, t.preds.ptr, t.labels.ptr, t.weights.ptr, t.rows,
                                    ctl, t.gmax_part.ptr, sampled ? t.samp_g.ptr : nullptr,
                                    sampled ? t.samp_h.ptr : nullptr));
    }
    if (sampled)
        MB_HIP(mbk::launch_sample(s, sample_params(t, tree), t.rows, ctl, t.goss_buckets.ptr,
                                  t.samp_g.ptr, t.samp_h.ptr, order,
                                  t.samp_h_kept.ptr, kept, plan, fixp,
                                  start_in_sample ? prev : nullptr,
                                  start_in_sample ? t.gmax_part.ptr : nullptr, walk_parts));
    else
        MB_HIP(mbk::launch_quantize(s, t.gp, t.preds.ptr, t.labels.ptr, t.weights.ptr, t.rows,
                                    ctl, order, implicit_rows, plan, fixp));
    return sampled;
}

// The walk that adds tree `tree` to the training predictions (and counts its
// deepest nodes' rows when count is non-null).  For single-output objectives
// without leaf renewal it also computes the next tree's gradient maxima (and
// g, h when that tree is sampled), so the next tree skips its own gradient
// pass over the predictions and labels.
static void training_walk(Trainer &t, int tree, const mbk::TreeOut &out, uint32_t *count,
                          const uint8_t *kept) {
    hipStream_t s = t.dev->stream;
    if (t.K == 1 && !t.renewal) {
        const bool next_sampled = tree_sampled(t.p, tree + 1);
        MB_HIP(mbk::launch_walk_count_grad(s, t.bins_fm.ptr, t.rows, t.nb, t.D, out, t.preds_cur,
                                           count, kept, t.gp, t.labels.ptr, t.weights.ptr,
                                           t.gmax_part.ptr, next_sampled ? t.samp_g.ptr : nullptr,
                                           next_sampled ? t.samp_h.ptr : nullptr,
                                           &t.walk_gparts));
    } else {
        MB_HIP(mbk::launch_walk_count(s, t.bins_fm.ptr, t.rows, t.nb, t.D, out,
                                      t.renewal ? nullptr : t.preds_cur, count, kept));
    }
}

static void grow_levelwise(Trainer &t, int tree) {
    hipStream_t s = t.dev->stream;
    const mbk::Shape &sh = t.sh;
    mbk::TreeOut out = t.tree_out(tree);
    if (const uint8_t *m = tree_feature_mask(t, tree))
        MB_HIP(hipMemcpyAsync(t.feat_mask.ptr, m, (size_t)t.cols, hipMemcpyHostToDevice, s));
    mbk::TreeCtl *ctl = t.ctl.ptr;
    // an unsampled root holds every row in order: its entries are the rows'
    // packed words only (row = entry index) until the first partition
    const bool sampled = tree_entries(t, tree, ctl, t.order_a.ptr,
                                      t.kept_walk ? t.kept.ptr : nullptr, true, out.cover);
    mbk::Entry *ord_cur = t.order_a.ptr, *ord_next = t.order_b.ptr;
    uint32_t *seg_cur = t.seg_a.ptr, *seg_next = t.seg_b.ptr;
    int64_t *h_cur = t.hist_a.ptr, *h_prev = t.hist_b.ptr;

    auto hist = [&](const mbk::Entry *ord, int level) {
        // profiling: the kernel's own dispatch timestamps (no marker packets)
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (t.prof_tree(tree)) {
            e0 = acquire_event();
            e1 = acquire_event();
        }
        // an unsampled root streams every row: the planar copy when there is one
        const bool planar = level == 0 && !sampled && t.has_root_copy;
        MB_HIP(mbk::launch_hist(s, planar ? t.sh_root : sh,
                                planar ? t.bins_root.ptr : t.bins_tiled.ptr, ord,
                                t.items.ptr, ctl, t.partials.ptr, t.hist_grid,
                                planar ? &t.root_layout : nullptr, e0, e1,
                                level == 0 && !sampled));
        if (e0) t.events.push_back({e0, e1, level});
    };
    const mbk::Shape &sh0 = !sampled && t.has_root_copy ? t.sh_root : sh;   // the root's

    // A level whose next partition is not the last one is decided inside that
    // partition (launch_route with RouteDecide) from the split search's keys:
    // one launch less per level.  The deepest split level keeps its decision
    // launch, which the final leaves and the walk read.
    const mbk::RouteDecide rd{t.split_keys.ptr, t.results.ptr, t.sp,       t.cols,
                              t.node_g.ptr,     t.node_h.ptr,  t.bounds.ptr, t.mono.ptr, ctl};
    auto split_level = [&](const mbk::Shape &shl, uint32_t pairs, const int64_t *hp, int64_t *hc,
                           const mbk::LevelArgs &la) {
        const bool fold = la.level + 1 < t.D;
        MB_HIP(mbk::launch_split(s, shl, t.sp, t.pairs.ptr, pairs, t.partials.ptr, hp, hc,
                                 t.is_cat.ptr, t.mono.ptr, t.feat_mask.ptr, ctl, t.count.ptr,
                                 t.node_g.ptr, t.node_h.ptr, la.level_start, t.results.ptr,
                                 fold ? t.split_keys.ptr : nullptr,
                                 fold ? t.route_cursor.ptr : nullptr));
        if (!fold)
            MB_HIP(mbk::launch_decide(s, sh, t.sp, la, t.results.ptr, t.count.ptr, t.node_g.ptr,
                                      t.node_h.ptr, t.bounds.ptr, t.mono.ptr, ctl,
                                      t.route_cursor.ptr, out));
    };

    // h = 1 for every row and no weights: every entry's quantised hessian is
    // 127, so a child's integer hessian sum orders children as its row count
    const int obj = t.p.objective;
    const bool unit_hess = !t.gp.has_weights && (obj == OBJ_L2 || obj == OBJ_MAE ||
                                                 obj == OBJ_HUBER || obj == OBJ_QUANTILE);

    // level 0
    hist(ord_cur, 0);
    split_level(sh0, 1, h_prev, h_cur, mbk::LevelArgs{0, 0, 1, 0});
    for (int d = 1; d <= t.D; ++d) {
        const bool terminal = d == t.D;
        mbk::LevelArgs lp{d - 1, (uint32_t)((1u << (d - 1)) - 1), 1u << (d - 1), terminal ? 1u : 0u};
        mbk::LevelArgs ln{d, (uint32_t)((1u << d) - 1), 1u << d, terminal ? 1u : 0u};
        if (terminal && (!sampled || t.kept_walk)) {
            // deepest level: leaf values, then one walk of the finished tree over
            // the training rows adds every row's leaf (the single addition the
            // partition-time update makes, route_samples apply,
            // Shaders.swift:1280-1311) and counts the deepest nodes' (kept) rows
            MB_HIP(mbk::launch_final_leaves(s, t.sp, ln, t.count.ptr, t.node_g.ptr, t.node_h.ptr,
                                            t.bounds.ptr, ctl, out, false));
            training_walk(t, tree, out, t.count.ptr, sampled ? t.kept.ptr : nullptr);
            if (!t.renewal && !t.has_valid) {
                // nothing of this tree reads the deepest covers or leaves
                // again before the next tree's root pass, which writes them
                // (the validation walk and leaf renewal below do)
                t.fix_pending = mbk::PendingFixup{ln, t.count.ptr, out, 1, 1};
                t.fix_tree = tree;
                break;
            }
            MB_HIP(mbk::launch_final_fixup(s, ln, t.count.ptr, out));
            if (t.renewal) {
                // residuals before the tree (routing applies nothing), then
                // one walk with the renewed leaves (Booster.swift:1596-1630)
                renew_tree(t, out, nullptr);
                MB_HIP(mbk::launch_predict_binned(s, t.bins_fm.ptr, t.rows, t.nb, t.D, out,
                                                  t.preds_cur));
            }
            break;
        }
        if (terminal) {
            // a sampled tree counts its kept rows with the partition; every
            // row's prediction then comes from one walk (Booster.swift:1568-1580)
            const mbk::RoutePlan rp = t.route_plan(ln, seg_next);
            MB_HIP(mbk::launch_route(s, sh, lp, t.bins_fm.ptr, ord_cur, ord_next, seg_cur,
                                     t.count.ptr, out, t.route_cursor.ptr,
                                     t.route_grid, false, &rp));
            MB_HIP(mbk::launch_final_leaves(s, t.sp, ln, t.count.ptr, t.node_g.ptr, t.node_h.ptr,
                                            t.bounds.ptr, ctl, out, true));
            if (t.renewal) renew_tree(t, out, nullptr);
            MB_HIP(mbk::launch_predict_binned(s, t.bins_fm.ptr, t.rows, t.nb, t.D, out,
                                              t.preds_cur));
            break;
        }
        // non-terminal here, so level d - 1 was decided by this partition's keys.
        // Before the deepest split level only the children that level builds
        // are read again (an unsampled tree's deepest rows are counted by the
        // walk), so only their entries are written when the hessian sums
        // name them.
        const mbk::RoutePlan rp = t.route_plan(ln, seg_next);
        const bool built_only = d == t.D - 1 && !sampled && unit_hess;
        MB_HIP(mbk::launch_route(s, sh, lp, t.bins_fm.ptr, ord_cur, ord_next, seg_cur,
                                 t.count.ptr, out, t.route_cursor.ptr, t.route_grid, true, &rp,
                                 d == 1 && !sampled, &rd, built_only));
        std::swap(ord_cur, ord_next);
        std::swap(seg_cur, seg_next);
        std::swap(h_cur, h_prev);
        hist(ord_cur, d);
        split_level(sh, 1u << (d - 1), h_prev, h_cur, ln);
    }
    if (t.has_valid)
        MB_HIP(mbk::launch_predict_binned(s, t.vbins_fm.ptr, t.vrows, t.nb, t.D, out,
                                          t.vpreds_cur));
    t.ctl_pending = tree;                            // copied by the next tree's start
}

static void finish_leafwise(Trainer &t, int tree, const mbk::TreeOut &out,
                            bool deep_counts = false);

// Best-first growth (growLeafWiseTree, Booster.swift:967-1310): root
// histogram and split, then numLeaves-1 steps of pick -> partition -> smaller
// child's histogram -> sibling by subtraction -> children's best splits.
static void grow_leafwise(Trainer &t, int tree) {
    hipStream_t s = t.dev->stream;
    const mbk::Shape &sh = t.sh;
    mbk::TreeOut out = t.tree_out(tree);
    if (const uint8_t *m = tree_feature_mask(t, tree))
        MB_HIP(hipMemcpyAsync(t.feat_mask.ptr, m, (size_t)t.cols, hipMemcpyHostToDevice, s));
    mbk::TreeCtl *ctl = t.ctl.ptr;
    mbk::Entry *order = t.order_a.ptr;
    const bool sampled = tree_entries(t, tree, ctl, order);
    const bool planar0 = !sampled && t.has_root_copy;
    const mbk::Shape &sh0 = planar0 ? t.sh_root : sh;   // the root's
    MB_HIP(mbk::launch_lw_init(s, sh0, t.lw, ctl, t.lw_state.ptr, t.lw_open.ptr, t.seg_a.ptr,
                               t.count.ptr, t.pairs.ptr, t.items.ptr, out,
                               sampled));
    auto build = [&](int step) {
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (t.prof_tree(tree)) {
            e0 = acquire_event();
            e1 = acquire_event();
        }
        const bool planar = step == 0 && !sampled && t.has_root_copy;
        const mbk::Shape &shs = planar ? sh0 : sh;
        MB_HIP(mbk::launch_hist(s, shs, planar ? t.bins_root.ptr : t.bins_tiled.ptr, order,
                                t.items.ptr, ctl, t.partials.ptr, t.hist_grid,
                                planar ? &t.root_layout : nullptr, e0, e1));
        if (e0) t.events.push_back({e0, e1, std::min(step, 15)});
        MB_HIP(mbk::launch_split(s, shs, t.sp, t.pairs.ptr, 1, t.partials.ptr, t.hist_a.ptr,
                                 t.hist_a.ptr, t.is_cat.ptr, t.mono.ptr, t.feat_mask.ptr, ctl,
                                 t.count.ptr, t.node_g.ptr, t.node_h.ptr, 0, t.results.ptr));
    };
    uint64_t *cursor = t.route_cursor.ptr;
    build(0);
    for (int it = 1; it < t.p.num_leaves; ++it) {
        // the previous build's leaves are evaluated inside the pick
        MB_HIP(mbk::launch_lw_pick(s, sh, t.sp, t.lw, t.lw_state.ptr, t.lw_open.ptr,
                                   t.results.ptr, t.node_g.ptr, t.node_h.ptr, t.mono.ptr, ctl,
                                   cursor, out));
        MB_HIP(mbk::launch_lw_partition(s, sh, t.lw, t.lw_state.ptr, t.lw_open.ptr, t.bins_fm.ptr,
                                        order, cursor, t.seg_a.ptr, t.count.ptr,
                                        ctl, t.pairs.ptr, t.items.ptr, out));
        build(it);
    }
    MB_HIP(mbk::launch_lw_eval(s, sh, t.sp, t.lw_state.ptr, t.lw_open.ptr, t.results.ptr,
                               t.node_g.ptr, t.node_h.ptr, ctl, out));
    if (t.renewal) MB_HIP(mbk::launch_lw_bounds(s, t.lw_state.ptr, t.lw_open.ptr, t.bounds.ptr));
    finish_leafwise(t, tree, out);
}

// A finished leaf-wise tree: training (and validation) predictions, leaf
// renewal, the tree's control block.  t.bounds holds every leaf's bounds.
// With deep_counts (no renewal) the walk also counts the rows of the
// depth-D nodes (zeroed before) and writes their covers.
static void finish_leafwise(Trainer &t, int tree, const mbk::TreeOut &out, bool deep_counts) {
    hipStream_t s = t.dev->stream;
    // training predictions: walk the finished tree on the binned rows
    // (predict_tree_binned, Shaders.swift:1763-1781); with leaf renewal the
    // renewed leaves are added after it
    if (t.renewal) {
        MB_HIP(mbk::launch_predict_binned(s, t.bins_fm.ptr, t.rows, t.nb, t.D, out, t.preds_cur));
    } else {
        training_walk(t, tree, out, deep_counts ? t.count.ptr : nullptr, nullptr);
        if (deep_counts) {
            // the depth-D covers, which nothing reads before the next tree's
            // root pass writes them (or the end of the grow call)
            const mbk::LevelArgs ld{t.D, (uint32_t)((1u << t.D) - 1), 1u << t.D, 1u};
            t.fix_pending = mbk::PendingFixup{ld, t.count.ptr, out, 0, 1};
            t.fix_tree = tree;
        }
    }
    if (t.has_valid)
        MB_HIP(mbk::launch_predict_binned(s, t.vbins_fm.ptr, t.vrows, t.nb, t.D, out,
                                          t.vpreds_cur));
    if (t.renewal) {
        // residuals after the tree's first leaf values, then each leaf's
        // change is added (Booster.swift:1253-1290)
        renew_tree(t, out, t.rn_delta.ptr);
        mbk::TreeOut dout = out;
        dout.leaf = t.rn_delta.ptr;
        MB_HIP(mbk::launch_predict_binned(s, t.bins_fm.ptr, t.rows, t.nb, t.D, dout,
                                          t.preds_cur));
        if (t.has_valid)
            MB_HIP(mbk::launch_predict_binned(s, t.vbins_fm.ptr, t.vrows, t.nb, t.D, dout,
                                              t.vpreds_cur));
    }
    t.ctl_pending = tree;                            // copied by the next tree's start
}

// Leaf-wise growth in depth rounds (trees of depth <= LWB_MAX_DEPTH): the
// level-wise chain of partition, planning, histograms and split search, over
// a speculative tree that each round's select kernel fills with the depth-r
// leaves the best-first loop may still pick (leaf_pick_apply and leaf_step,
// Shaders.swift:720-1091); the select kernels write the picked nodes into
// the tree, so it equals the one-leaf-per-step tree.
static void grow_leafwise_rounds(Trainer &t, int tree) {
    hipStream_t s = t.dev->stream;
    const mbk::Shape &sh = t.sh;
    mbk::TreeOut out = t.tree_out(tree);
    if (const uint8_t *m = tree_feature_mask(t, tree))
        MB_HIP(hipMemcpyAsync(t.feat_mask.ptr, m, (size_t)t.cols, hipMemcpyHostToDevice, s));
    mbk::TreeCtl *ctl = t.ctl.ptr;
    mbk::TreeOut spec{t.spec_split.ptr, t.spec_cover.ptr, t.spec_cover.ptr, t.spec_cover.ptr,
                      t.spec_mask.ptr};
    const bool sampled = tree_entries(t, tree, ctl, t.order_a.ptr, nullptr, false, spec.cover);
    // the two halves of the leaf-wise order buffer alternate by depth
    mbk::Entry *ord_cur = t.order_a.ptr, *ord_next = t.order_a.ptr + t.rows;
    uint32_t *seg_cur = t.seg_a.ptr, *seg_next = t.seg_b.ptr;
    int64_t *h_cur = t.hist_a.ptr, *h_prev = t.hist_b.ptr;
    auto hist = [&](const mbk::Entry *ord, int level) {
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (t.prof_tree(tree)) {
            e0 = acquire_event();
            e1 = acquire_event();
        }
        const bool planar = level == 0 && !sampled && t.has_root_copy;
        MB_HIP(mbk::launch_hist(s, planar ? t.sh_root : sh,
                                planar ? t.bins_root.ptr : t.bins_tiled.ptr, ord,
                                t.items.ptr, ctl, t.partials.ptr, t.hist_grid,
                                planar ? &t.root_layout : nullptr, e0, e1));
        if (e0) t.events.push_back({e0, e1, level});
    };
    const mbk::Shape &sh0 = !sampled && t.has_root_copy ? t.sh_root : sh;   // the root's
    // unsampled trees without renewal: the training walk counts the deepest
    // rows, so the last round partitions nothing
    mbk::LWBArgs la = t.lwb;
    la.deep_walk = !sampled && !t.renewal ? 1 : 0;
    auto select = [&](int round) {
        MB_HIP(mbk::launch_lwb_select(s, sh, t.sp, la, round, t.results.ptr, t.count.ptr,
                                      t.node_g.ptr, t.node_h.ptr, t.bounds.ptr, t.mono.ptr, ctl,
                                      t.route_cursor.ptr, t.lwb_state.ptr, t.lwb_cand.ptr, spec,
                                      out));
    };
    hist(ord_cur, 0);
    MB_HIP(mbk::launch_split(s, sh0, t.sp, t.pairs.ptr, 1, t.partials.ptr, h_prev, h_cur,
                             t.is_cat.ptr, t.mono.ptr, t.feat_mask.ptr, ctl, t.count.ptr,
                             t.node_g.ptr, t.node_h.ptr, 0, t.results.ptr));
    for (int r = 0; r < t.D; ++r) {
        const bool last = r + 1 == t.D;
        select(r);
        if (last && la.deep_walk) break;
        mbk::LevelArgs lp{r, (uint32_t)((1u << r) - 1), 1u << r, last ? 1u : 0u};
        mbk::LevelArgs ln{r + 1, (uint32_t)((1u << (r + 1)) - 1), 1u << (r + 1), last ? 1u : 0u};
        // the deepest children are never evaluated: count them, move nothing
        const mbk::RoutePlan rp = t.route_plan(ln, seg_next);
        MB_HIP(mbk::launch_route(s, sh, lp, t.bins_fm.ptr, ord_cur, ord_next, seg_cur,
                                 t.count.ptr, spec, t.route_cursor.ptr, t.route_grid, !last, &rp));
        if (last) break;
        std::swap(ord_cur, ord_next);
        std::swap(seg_cur, seg_next);
        std::swap(h_cur, h_prev);
        hist(ord_cur, r + 1);
        MB_HIP(mbk::launch_split(s, sh, t.sp, t.pairs.ptr, 1u << r, t.partials.ptr, h_prev, h_cur,
                                 t.is_cat.ptr, t.mono.ptr, t.feat_mask.ptr, ctl, t.count.ptr,
                                 t.node_g.ptr, t.node_h.ptr, ln.level_start, t.results.ptr));
    }
    select(t.D);
    finish_leafwise(t, tree, out, la.deep_walk != 0);
}

void trainer_grow(Trainer *tp, int num_trees) {
    Phase ph("grow trees");
    Trainer &t = *tp;
    hipStream_t s = t.dev->stream;
    t.ensure_capacity(t.grown + num_trees);
    const int first_tree = t.grown;
    const bool metric_each_tree = t.has_valid;
    std::vector<float> vp;
    const int K = t.K;
    auto metric = [&](const float *pred, const float *y, int64_t n) {
        return K > 1 ? multiclass_logloss(pred, y, n, K) : eval_metric(t.p, pred, y, n);
    };
    for (int k = 0; k < num_trees && !t.stopped; ++k) {
        const int tree = t.grown;
        // tree t fits class t % K (Booster.swift:1315)
        const int cls = tree % K;
        t.gp.class_index = cls;
        t.preds_cur = t.preds.ptr + (size_t)cls * (size_t)t.rows;
        t.vpreds_cur = t.has_valid ? t.vpreds.ptr + (size_t)cls * (size_t)t.vrows : nullptr;
        if (t.lw_rounds) grow_leafwise_rounds(t, tree);
        else if (t.leafwise) grow_leafwise(t, tree);
        else grow_levelwise(t, tree);
        t.grown += 1;
        // metrics once per round of K trees (Booster.swift:1650-1688)
        if (t.grown % K != 0) continue;
        const int round = t.grown / K;
        const bool is_last = k + 1 == num_trees;
        const bool log_now = t.p.eval_every > 0 && (round % t.p.eval_every == 0 || is_last);
        if (!metric_each_tree && !log_now) continue;
        MB_HIP(hipStreamSynchronize(s));
        std::string line;
        if (log_now) {
            std::vector<float> tp_h((size_t)t.rows * (size_t)K);
            MB_HIP(hipMemcpy(tp_h.data(), t.preds.ptr, tp_h.size() * 4, hipMemcpyDeviceToHost));
            if (t.labels_h.empty()) {
                t.labels_h.resize((size_t)t.rows);
                MB_HIP(hipMemcpy(t.labels_h.data(), t.labels.ptr, t.labels_h.size() * 4,
                                 hipMemcpyDeviceToHost));
            }
            char buf[128];
            std::snprintf(buf, sizeof buf, "[%4d] train-%s: %.5f", round,
                          effective_metric(t.p).c_str(),
                          metric(tp_h.data(), t.labels_h.data(), t.rows));
            line = buf;
        }
        if (t.has_valid) {
            vp.resize((size_t)t.vrows * (size_t)K);
            MB_HIP(hipMemcpy(vp.data(), t.vpreds.ptr, vp.size() * 4, hipMemcpyDeviceToHost));
            const float vm = metric(vp.data(), t.vlabels_h.data(), t.vrows);
            t.eval_history.push_back(vm);
            const bool higher = effective_metric(t.p) == "auc";
            if (higher ? vm > t.best_metric : vm < t.best_metric) {
                t.best_metric = vm;
                t.best_iter = round;
                t.stale = 0;
            } else {
                t.stale += 1;
            }
            if (log_now) {
                char buf[96];
                std::snprintf(buf, sizeof buf, "   valid-%s: %.5f", effective_metric(t.p).c_str(), vm);
                line += buf;
            }
            if (t.p.early_stopping_rounds > 0 && t.stale >= t.p.early_stopping_rounds) {
                if (t.p.verbose && !line.empty()) std::printf("%s\n", line.c_str());
                if (t.p.verbose)
                    std::printf("early stopping at iteration %d (best: %d, valid-%s %.5f)\n", round,
                                t.best_iter, effective_metric(t.p).c_str(), t.best_metric);
                t.stopped = true;
                break;
            }
        }
        if (t.p.verbose && !line.empty()) std::printf("%s\n", line.c_str());
    }
    if (t.fix_pending.active) {                      // the last tree's deepest covers
        const mbk::PendingFixup &f = t.fix_pending;
        MB_HIP(mbk::launch_final_fixup(s, f.la, f.count, t.tree_out(t.fix_tree),
                                       f.zero_empty != 0));
        t.fix_pending.active = 0;
    }
    if (t.ctl_pending >= 0) {                        // the last tree's control block
        MB_HIP(hipMemcpyAsync(t.ctl_hist.ptr + t.ctl_pending, t.ctl.ptr, sizeof(mbk::TreeCtl),
                              hipMemcpyDeviceToDevice, s));
        t.ctl_pending = -1;
    }
    MB_HIP(hipStreamSynchronize(s));
    if (t.grown > first_tree) {
        std::vector<mbk::TreeCtl> c((size_t)(t.grown - first_tree));
        MB_HIP(hipMemcpy(c.data(), t.ctl_hist.ptr + first_tree, c.size() * sizeof(mbk::TreeCtl),
                         hipMemcpyDeviceToHost));
        for (const auto &e : c)
            if (e.overflow == mbk::LWB_MISSED_PICK)
                internal("leaf-wise rounds: a picked leaf was never expanded");
            else if (e.overflow) internal("histogram item list overflow");
    }
    if (t.profiling) {
        for (auto &e : t.events) {
            float ms = 0;
            MB_HIP(hipEventElapsedTime(&ms, e.start, e.end));
            t.prof_ms += ms;
            t.prof_level_ms[e.level & 15] += ms;
            t.prof_launches += 1;
            release_event(e.start);
            release_event(e.end);
        }
        t.events.clear();
    }
}

void trainer_profile(Trainer *t, int every) {
    if (every > 0 && !t->profiling) {
        t->prof_first_tree = t->grown;
        t->prof_every = every;
        t->prof_ms = 0;
        t->prof_launches = 0;
        for (double &v : t->prof_level_ms) v = 0;
    }
    t->profiling = every > 0;
}

// The control blocks of the profiled trees since profiling began.
static std::vector<mbk::TreeCtl> profiled_ctls(Trainer *t) {
    std::vector<mbk::TreeCtl> out;
    const int n = t->grown - t->prof_first_tree;
    if (n <= 0) return out;
    std::vector<mbk::TreeCtl> h((size_t)n);
    MB_HIP(hipMemcpy(h.data(), t->ctl_hist.ptr + t->prof_first_tree, (size_t)n * sizeof(mbk::TreeCtl),
                     hipMemcpyDeviceToHost));
    for (int k = 0; k < n; k += t->prof_every) out.push_back(h[(size_t)k]);
    return out;
}

void trainer_hist_stats(Trainer *t, int64_t *launches, double *ms, double *bytes) {
    MB_HIP(hipStreamSynchronize(t->dev->stream));
    double b = 0;
    for (const auto &c : profiled_ctls(t))
        for (int d = 0; d < t->D; ++d) b += (double)c.level_built[d] * (double)(t->cols + 4);
    if (launches) *launches = t->prof_launches;
    if (ms) *ms = t->prof_ms;
    if (bytes) *bytes = b;
}

void trainer_level_stats(Trainer *t, int32_t max_levels, int64_t *built, int64_t *active,
                         double *hist_ms) {
    MB_HIP(hipStreamSynchronize(t->dev->stream));
    for (int d = 0; d < max_levels; ++d) {
        if (built) built[d] = 0;
        if (active) active[d] = 0;
        if (hist_ms) hist_ms[d] = d < 16 ? t->prof_level_ms[d] : 0.0;
    }
    const int L = std::min<int>(max_levels, 16);
    for (const auto &c : profiled_ctls(t))
        for (int d = 0; d < L; ++d) {
            if (built) built[d] += c.level_built[d];
            if (active) active[d] += c.level_active[d];
        }
}

void trainer_setup_seconds(Trainer *t, double *edges_s, double *bin_s) {
    if (edges_s) *edges_s = t->t_edges;
    if (bin_s) *bin_s = t->t_bin;
}

// Read finished trees back (drainPending, Booster.swift:903-948): reachable
// nodes only, numeric thresholds from the bin edges.
Booster *trainer_booster(Trainer *tp) {
    Phase ph("model readback");
    Trainer &t = *tp;
    MB_HIP(hipStreamSynchronize(t.dev->stream));
    const int n = t.grown;
    const size_t tn = (size_t)t.total_nodes;
    std::vector<mbk::NodeSplit> sp((size_t)n * tn);
    std::vector<float> leaf((size_t)n * tn), gain((size_t)n * tn), cover((size_t)n * tn);
    std::vector<uint32_t> mask((size_t)n * tn * 8);
    if (n > 0) {
        MB_HIP(hipMemcpy(sp.data(), t.m_split.ptr, sp.size() * sizeof(mbk::NodeSplit), hipMemcpyDeviceToHost));
        MB_HIP(hipMemcpy(leaf.data(), t.m_leaf.ptr, leaf.size() * 4, hipMemcpyDeviceToHost));
        MB_HIP(hipMemcpy(gain.data(), t.m_gain.ptr, gain.size() * 4, hipMemcpyDeviceToHost));
        MB_HIP(hipMemcpy(cover.data(), t.m_cover.ptr, cover.size() * 4, hipMemcpyDeviceToHost));
        MB_HIP(hipMemcpy(mask.data(), t.m_mask.ptr, mask.size() * 4, hipMemcpyDeviceToHost));
    }
    auto b = std::make_unique<Booster>();
    b->params = t.user_params;
    b->num_features = t.cols;
    b->has_feature_names = t.has_feature_names;
    b->feature_names = t.feature_names;
    b->trained_num_bins = t.nb;
    b->trained_categorical = t.p.categorical;
    b->base_score = t.base;
    b->base_scores = t.base_scores;
    b->trained_num_classes = t.K;
    b->warnings = t.warnings;
    b->eval_history = t.eval_history;
    const int data_bins = t.nb - 1;
    int keep = n;
    if (t.has_valid) {
        b->best_iteration = t.best_iter;
        if (t.p.early_stopping_rounds > 0 && keep > t.best_iter * t.K) keep = t.best_iter * t.K;
    }
    b->trees = t.init_trees;
    b->trees.reserve(t.init_trees.size() + (size_t)keep);
    for (int k = 0; k < keep; ++k) {
        Tree tr;
        tr.feature.assign(tn, -1);
        tr.threshold.assign(tn, 0.0f);
        tr.leaf.assign(tn, 0.0f);
        tr.flags.assign(tn, 0);
        if (t.has_cats) tr.cat_mask.assign(tn * 8, 0u);
        tr.gain.assign(tn, 0.0f);
        tr.cover.assign(tn, 0.0f);
        const size_t base_n = (size_t)k * tn;
        std::vector<int> stack{0};
        while (!stack.empty()) {
            int nd = stack.back();
            stack.pop_back();
            const mbk::NodeSplit &s = sp[base_n + nd];
            tr.cover[nd] = cover[base_n + nd];
            if (s.feature >= 0) {
                tr.feature[nd] = s.feature;
                tr.flags[nd] = (uint8_t)s.flags;
                tr.gain[nd] = gain[base_n + nd];
                if (s.flags & mbk::FLAG_CATEGORICAL) {
                    if (t.has_cats)
                        for (int w = 0; w < 8; ++w)
                            tr.cat_mask[(size_t)nd * 8 + w] = mask[(base_n + nd) * 8 + w];
                } else {
                    tr.threshold[nd] = t.edges[(size_t)s.feature * (data_bins - 1) + s.bin];
                }
                stack.push_back(2 * nd + 1);
                stack.push_back(2 * nd + 2);
            } else {
                tr.leaf[nd] = leaf[base_n + nd];
            }
        }
        b->trees.push_back(std::move(tr));
    }
    return b.release();
}

void trainer_free(Trainer *t) {
    Phase ph("release trainer");
    delete t;
}

int trainer_classes(const Trainer *t) { return t->K; }

}  // namespace mb
