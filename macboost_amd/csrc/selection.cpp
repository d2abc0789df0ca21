// selection.cpp — Boruta feature selection (FeatureSelection.swift:45-203):
// each round trains a disposable model on the binned features plus row-
// permuted shadow copies built on the device, and votes every real feature's
// gain importance against the best shadow's.
#include <cmath>

#include "core.hpp"

namespace mb {

namespace {

// P[Binomial(rounds, 0.5) >= k] by the pmf recurrence (FeatureSelection.swift:193-203).
double binomial_tail(int k, int rounds) {
    if (k <= 0) return 1.0;
    double pmf = std::pow(0.5, (double)rounds), tail = 0.0;
    for (int i = 0; i <= rounds; ++i) {
        if (i >= k) tail += pmf;
        if (i < rounds) pmf *= (double)(rounds - i) / (double)(i + 1);
    }
    return std::min(1.0, tail);
}

}  // namespace

SelectionResult select_features(const Params &p, const float *x, int64_t rows, int64_t cols,
                                const float *y, const float *w, int rounds, int trees,
                                double alpha, uint64_t seed) {
    validate_params(p);
    if (rounds < 5) invalid("selection needs rounds >= 5 for the binomial test");
    if (!(alpha > 0 && alpha < 1)) invalid("alpha must be in (0, 1)");
    if (rows > 0xFFFFFFF0LL) invalid("more than 2^32 rows are not supported");
    validate_label_values(p, y, rows);
    validate_categoricals(p, x, rows, cols, 1, rows);

    // bin the real features once (edges and bins on the device)
    Device dev(0);
    hipStream_t s = dev.stream;
    std::vector<uint8_t> is_cat((size_t)cols, 0);
    for (int f : p.categorical) is_cat[(size_t)f] = 1;
    const size_t ne = (size_t)p.num_bins - 2;
    DevBuf<float> xd((size_t)rows * (size_t)cols), ed(std::max<size_t>(1, (size_t)cols * ne));
    DevBuf<uint8_t> cat((size_t)cols), fm((size_t)rows * (size_t)cols);
    DevBuf<uint8_t> fm2((size_t)rows * 2 * (size_t)cols);
    MB_HIP(hipMemcpyAsync(cat.ptr, is_cat.data(), (size_t)cols, hipMemcpyHostToDevice, s));
    upload(xd.ptr, x, xd.bytes(), s);
    {
        const size_t cap = mbk::edge_sample_cap(rows);
        DevBuf<uint32_t> ka((size_t)cols * cap), kb((size_t)cols * cap), cnt((size_t)cols);
        MB_HIP(mbk::launch_edges(s, xd.ptr, rows, (int)cols, 1, rows, p.num_bins, cat.ptr, ka.ptr,
                                 kb.ptr, cnt.ptr, ed.ptr));
        DevBuf<uint8_t> tiled((size_t)rows * 8);     // scratch: the 8-wide gather output
        for (int64_t f0 = 0; f0 < cols; f0 += 8) {
            const int n = (int)std::min<int64_t>(8, cols - f0);
            MB_HIP(mbk::launch_bin_data(s, xd.ptr + f0 * rows, rows, n, 1, rows,
                                        ed.ptr + f0 * (int64_t)ne, cat.ptr + f0, p.num_bins, 8, 1,
                                        tiled.ptr, fm.ptr + f0 * rows));
        }
        MB_HIP(hipStreamSynchronize(s));
    }
    std::vector<float> edges((size_t)cols * ne);
    if (!edges.empty())
        MB_HIP(hipMemcpy(edges.data(), ed.ptr, edges.size() * 4, hipMemcpyDeviceToHost));
    std::vector<float> edges2 = edges;
    edges2.insert(edges2.end(), edges.begin(), edges.end());

    Params sp = p;                                   // the disposable probe models
    sp.has_monotone = false;
    sp.monotone.clear();
    sp.has_allowed = false;
    sp.allowed.clear();
    for (int f : p.categorical) sp.categorical.insert(f + (int)cols);
    sp.num_trees = trees > 0 ? trees : std::min(p.num_trees, 100);
    sp.early_stopping_rounds = 0;
    sp.eval_every = 0;
    sp.init_model.clear();

    int bits = 1;
    while (((int64_t)1 << bits) < rows) ++bits;
    const uint32_t half_bits = (uint32_t)((bits + 1) / 2);
    std::vector<int32_t> hits((size_t)cols, 0);
    std::vector<double> gain_sum((size_t)cols, 0.0);
    double shadow_sum = 0.0;
    for (int r = 0; r < rounds; ++r) {
        const uint32_t round_seed = (uint32_t)(seed + (uint64_t)r * 0x9E3779B97F4A7C15ULL + 1u);
        MB_HIP(mbk::launch_shadow_bins(s, fm.ptr, rows, (int)cols, half_bits, round_seed, fm2.ptr));
        MB_HIP(hipStreamSynchronize(s));
        std::unique_ptr<Trainer, void (*)(Trainer *)> t(
            trainer_create_fm(sp, rows, 2 * cols, fm2.ptr, edges2, y, w), trainer_free);
        trainer_grow(t.get(), sp.num_trees * trainer_classes(t.get()));
        std::unique_ptr<Booster> b(trainer_booster(t.get()));
        const std::vector<float> g = b->feature_importance(0);
        float mx = 0.0f;
        for (int64_t f = cols; f < 2 * cols; ++f) mx = f == cols ? g[(size_t)f] : std::max(mx, g[(size_t)f]);
        for (int64_t f = 0; f < cols; ++f) {
            if (g[(size_t)f] > mx) hits[(size_t)f] += 1;
            gain_sum[(size_t)f] += (double)g[(size_t)f];
        }
        shadow_sum += (double)mx;
        if (p.verbose) {
            int leading = 0;
            for (int32_t h : hits) leading += h == r + 1;
            std::printf("[Selection] round %d/%d: %d features beat every shadow so far\n", r + 1,
                        rounds, leading);
        }
    }
    SelectionResult res;
    res.hits = hits;
    res.decision.assign((size_t)cols, 1);
    res.gain_ratio.resize((size_t)cols);
    const double cutoff = alpha / (double)cols;
    for (int64_t f = 0; f < cols; ++f) {
        if (binomial_tail(hits[(size_t)f], rounds) < cutoff) res.decision[(size_t)f] = 2;
        else if (binomial_tail(rounds - hits[(size_t)f], rounds) < cutoff) res.decision[(size_t)f] = 0;
        res.gain_ratio[(size_t)f] =
            (float)(gain_sum[(size_t)f] / std::max(shadow_sum, 2.2250738585072014e-308));
    }
    return res;
}

}  // namespace mb
