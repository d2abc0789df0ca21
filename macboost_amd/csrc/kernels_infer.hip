// kernels_infer.hip — gfx950 inference kernels: batch forest prediction on raw
// features (predict_forest, Shaders.swift:1541-1584), the binned single-tree
// walk used for per-iteration validation (predict_tree_binned, :1763-1781) and
// exact TreeSHAP (gpu_treeshap, :1656-1734).
//
// TreeSHAP here gives each row a wavefront and each root-to-leaf path a lane,
// extending/unwinding in double precision and accumulating the row's phi in
// LDS (the wavefront owns it, so the summation order is fixed), with a single
// rounding to f32 at the end.
#include <algorithm>

#include "grad.h"
#include "mbk.h"

#include <math.h>

namespace mbk {

__device__ __forceinline__ bool raw_goes_left(float v, uint32_t flags, float thr,
                                              const uint32_t *mask_node, int32_t data_bins) {
    if (flags & FLAG_CATEGORICAL) {
        uint32_t cat = (uint32_t)data_bins;            // unseen -> missing
        if (isfinite(v)) {
            const float r = rintf(v);
            if (r >= 0.0f && (int64_t)r < data_bins) cat = (uint32_t)r;
        }
        return mask_node ? ((mask_node[cat >> 5] >> (cat & 31u)) & 1u) != 0 : false;
    }
    if (isnan(v)) return (flags & FLAG_DEFAULT_LEFT) != 0;
    return v <= thr;
}

__global__ __launch_bounds__(256) void k_predict_forest(ForestDev f, const float *__restrict__ x,
                                                        int64_t rows, int32_t data_bins, float base,
                                                        float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    float acc = base;                                  // seeded with the base, trees in order
    for (int32_t t = f.tree_first; t < f.num_trees; t += f.tree_step) {
        const int64_t b = (int64_t)t * f.nodes_per_tree;
        int32_t n = 0;
        int32_t feat = f.feature[b];
        while (feat >= 0) {
            const float v = x[(int64_t)feat * rows + i];
            const bool left = raw_goes_left(v, f.flags[b + n], f.threshold[b + n],
                                            f.mask ? f.mask + (b + n) * 8 : nullptr, data_bins);
            n = 2 * n + 1 + (left ? 0 : 1);
            feat = f.feature[b + n];
        }
        acc += f.leaf[b + n];
    }
    out[i * f.out_stride] = acc;
}

hipError_t launch_predict_forest(hipStream_t s, const ForestDev &f, const float *x, int64_t rows,
                                 int32_t data_bins, float base, float *out) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_predict_forest, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, f,
                       x, rows, data_bins, base, out);
    return hipGetLastError();
}

// Compute units of the current device (cached per device id).
static int device_cus() {
    static int cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// The same walk over the training rows, eight rows per thread walked level by
// level together, that also counts the rows reaching each node of the deepest
// level (counters in LDS, one global add per non-empty node per block).  The
// split records (feature, bin | flags << 8) and leaf values are staged in LDS,
// so each level costs one global gather per row: the row's bin byte.
// With GRAD the walk also starts the next tree's gradient pass on the updated
// predictions: per-block maxima of |g| and h into gpart (as k_grad_max's
// partials) and, with g_out / h_out, every row's g and h.
constexpr int WALK_THREADS = 1024;
constexpr int WALK_ROWS = 8;

struct WalkGrad {
    GradParams gp;
    const float *labels;
    const float *weights;
    uint32_t *gpart;
    float *g_out, *h_out;
};

template <bool GRAD>
__global__ __launch_bounds__(WALK_THREADS, 8) void k_walk_count(const uint8_t *__restrict__ bins_fm,
                                                             int64_t rows, int32_t nb,
                                                             int32_t max_depth, TreeOut tree,
                                                             float *__restrict__ preds,
                                                             uint32_t *__restrict__ count,
                                                             const uint8_t *__restrict__ kept,
                                                             WalkGrad wg) {
    extern __shared__ uint32_t wc_lds[];
    const uint32_t deep = 1u << max_depth, deep_start = deep - 1;
    const uint32_t internal = deep - 1, total = 2 * deep - 1;
    uint32_t *s_cnt = wc_lds;                        // [deep]
    int32_t *s_feat = reinterpret_cast<int32_t *>(wc_lds + deep);    // [internal]
    uint32_t *s_bf = wc_lds + deep + internal;       // [internal] bin | flags << 8
    float *s_leaf = reinterpret_cast<float *>(wc_lds + deep + 2 * internal);   // [total]
    for (uint32_t k = threadIdx.x; k < deep; k += blockDim.x) s_cnt[k] = 0;
    for (uint32_t k = threadIdx.x; k < internal; k += blockDim.x) {
        const NodeSplit s = tree.split[k];
        s_feat[k] = s.feature;
        s_bf[k] = (s.bin & 0xFFu) | ((s.flags & 0xFFu) << 8);
    }
    for (uint32_t k = threadIdx.x; k < total; k += blockDim.x) s_leaf[k] = tree.leaf[k];
    __syncthreads();
    constexpr int64_t CHUNK = (int64_t)WALK_THREADS * WALK_ROWS;
    uint32_t mg = 0, mh = 0;
    for (int64_t c0 = (int64_t)blockIdx.x * CHUNK; c0 < rows; c0 += (int64_t)gridDim.x * CHUNK) {
        const int64_t base = c0 + threadIdx.x;
        uint32_t n[WALK_ROWS];
#pragma unroll
        for (int k = 0; k < WALK_ROWS; ++k) n[k] = 0;
        // which rows count, loaded up front with the first level's bins
        uint32_t counts = count ? (1u << WALK_ROWS) - 1u : 0u;
        if (count && kept) {
#pragma unroll
            for (int k = 0; k < WALK_ROWS; ++k) {
                const int64_t i = base + (int64_t)k * WALK_THREADS;
                if (i < rows && !kept[i]) counts &= ~(1u << k);
            }
        }
        for (int32_t d = 0; d < max_depth; ++d) {
            uint32_t b[WALK_ROWS];
#pragma unroll
            for (int k = 0; k < WALK_ROWS; ++k) {
                const int64_t i = base + (int64_t)k * WALK_THREADS;
                const int32_t f = n[k] < internal ? s_feat[n[k]] : -1;
                b[k] = (i < rows && f >= 0) ? bins_fm[(int64_t)f * rows + i] : 0xFFFFFFFFu;
            }
#pragma unroll
            for (int k = 0; k < WALK_ROWS; ++k) {
                if (b[k] == 0xFFFFFFFFu) continue;   // past the end, or at a leaf
                const uint32_t bf = s_bf[n[k]], bin = bf & 0xFFu, flags = bf >> 8;
                bool left;
                if (flags & FLAG_CATEGORICAL)
                    left = ((tree.mask[n[k] * 8 + (b[k] >> 5)] >> (b[k] & 31u)) & 1u) != 0;
                else if (b[k] == (uint32_t)(nb - 1)) left = (flags & FLAG_DEFAULT_LEFT) != 0;
                else left = b[k] <= bin;
                n[k] = 2 * n[k] + 1 + (left ? 0 : 1);
            }
        }
#pragma unroll
        for (int k = 0; k < WALK_ROWS; ++k) {
            const int64_t i = base + (int64_t)k * WALK_THREADS;
            if (i >= rows) continue;
            if (preds) {                             // null: counts only
                const float np = preds[i] + s_leaf[n[k]];
                preds[i] = np;
                if (GRAD) {
                    float g, h;
                    const float w = wg.gp.has_weights ? wg.weights[i] : 1.0f;
                    row_grad(wg.gp, np, wg.labels[i], w, g, h);
                    mg = max(mg, __float_as_uint(fabsf(g)));
                    mh = max(mh, __float_as_uint(h));
                    if (wg.g_out) { wg.g_out[i] = g; wg.h_out[i] = h; }
                }
            }
            if (((counts >> k) & 1u) && n[k] >= deep_start) atomicAdd(&s_cnt[n[k] - deep_start], 1u);
        }
    }
    if (GRAD) {
        __shared__ uint32_t red[2][WALK_THREADS / 64];
        for (int o = 32; o > 0; o >>= 1) {
            mg = max(mg, (uint32_t)__shfl_xor((int)mg, o, 64));
            mh = max(mh, (uint32_t)__shfl_xor((int)mh, o, 64));
        }
        if ((threadIdx.x & 63) == 0) { red[0][threadIdx.x >> 6] = mg; red[1][threadIdx.x >> 6] = mh; }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t a = red[0][0], b = red[1][0];
            for (int k = 1; k < WALK_THREADS / 64; ++k) { a = max(a, red[0][k]); b = max(b, red[1][k]); }
            wg.gpart[2 * blockIdx.x] = a;
            wg.gpart[2 * blockIdx.x + 1] = b;
        }
    }
    if (!count) return;                              // null: predictions only
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < deep; k += blockDim.x)
        if (s_cnt[k]) atomicAdd(&count[deep_start + k], s_cnt[k]);
}

static int64_t walk_grid(int64_t rows) {
    const int64_t per = (int64_t)WALK_THREADS * WALK_ROWS;
    // two 1024-thread blocks per CU, or one block per chunk when fewer
    return std::max<int64_t>(1, std::min<int64_t>((rows + per - 1) / per, 2 * (int64_t)device_cus()));
}

hipError_t launch_walk_count(hipStream_t s, const uint8_t *bins_fm, int64_t rows,
                             int32_t num_bins, int32_t max_depth, const TreeOut tree,
                             float *preds, uint32_t *count, const uint8_t *kept) {
    if (rows <= 0) return hipSuccess;
    const size_t deep = (size_t)1 << max_depth;
    const size_t lds = (deep + 2 * (deep - 1) + (2 * deep - 1)) * sizeof(uint32_t);
    hipLaunchKernelGGL(k_walk_count<false>, dim3((unsigned)walk_grid(rows)), dim3(WALK_THREADS),
                       lds, s, bins_fm, rows, num_bins, max_depth, tree, preds, count, kept,
                       WalkGrad{});
    return hipGetLastError();
}

hipError_t launch_walk_count_grad(hipStream_t s, const uint8_t *bins_fm, int64_t rows,
                                  int32_t num_bins, int32_t max_depth, const TreeOut tree,
                                  float *preds, uint32_t *count, const uint8_t *kept,
                                  const GradParams &gp, const float *labels,
                                  const float *weights, uint32_t *gpart, float *g_out,
                                  float *h_out, int *partials) {
    *partials = 0;
    if (rows <= 0 || !preds) return hipErrorInvalidValue;
    if (gp.objective == 7) return hipErrorInvalidValue;   // one output per row only
    const size_t deep = (size_t)1 << max_depth;
    const size_t lds = (deep + 2 * (deep - 1) + (2 * deep - 1)) * sizeof(uint32_t);
    const int64_t grid = walk_grid(rows);
    hipLaunchKernelGGL(k_walk_count<true>, dim3((unsigned)grid), dim3(WALK_THREADS), lds, s,
                       bins_fm, rows, num_bins, max_depth, tree, preds, count, kept,
                       WalkGrad{gp, labels, weights, gpart, g_out, h_out});
    *partials = (int)grid;
    return hipGetLastError();
}

// Binned single-tree prediction (predict_tree_binned, Shaders.swift:1763-1781):
// the same walk with the tree staged in LDS, without counts.
hipError_t launch_predict_binned(hipStream_t s, const uint8_t *bins_fm, int64_t rows,
                                 int32_t num_bins, int32_t max_depth, const TreeOut tree,
                                 float *preds) {
    return launch_walk_count(s, bins_fm, rows, num_bins, max_depth, tree, preds, nullptr, nullptr);
}

// ---------------------------------------------------------------------------
// TreeSHAP
// ---------------------------------------------------------------------------

constexpr int SHAP_MAX_U = 12;                         // maxDepth <= 12

// Lane-per-row TreeSHAP for wide data (more columns than k_treeshap_rows
// keeps in LDS): every lane walks all paths for its row, phi in a global
// [blocks][cols][64] fp64 scratch.
__global__ __launch_bounds__(64) void k_treeshap(const float *__restrict__ x, int64_t rows,
                                                 int32_t cols, int32_t data_bins,
                                                 const uint32_t *__restrict__ masks,
                                                 const ShapPath *__restrict__ paths,
                                                 int32_t num_paths,
                                                 const ShapElem *__restrict__ elems,
                                                 const ShapUniq *__restrict__ uniq, float bias,
                                                 float *__restrict__ out,
                                                 double *__restrict__ phi_global) {
    const int lane = threadIdx.x;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    const bool valid = i < rows;
    const int64_t irow = valid ? i : 0;
    double *phi = phi_global + (int64_t)blockIdx.x * 64 * cols;   // this block's [cols][64]
    for (int f = 0; f < cols; ++f) phi[f * 64 + lane] = 0.0;
    for (int32_t p = 0; p < num_paths; ++p) {
        const ShapPath P = paths[p];
        double one[SHAP_MAX_U], zero[SHAP_MAX_U];
        int feat[SHAP_MAX_U];
#pragma unroll
        for (int u = 0; u < SHAP_MAX_U; ++u) {
            one[u] = 1.0;
            zero[u] = 1.0;
            feat[u] = 0;
            if (u < P.num_uniq) {
                const ShapUniq q = uniq[P.uniq_start + u];
                zero[u] = q.zero;
                feat[u] = q.feature;
            }
        }
        for (int e = 0; e < P.num_elem; ++e) {
            const ShapElem el = elems[P.elem_start + e];
            const float v = x[(int64_t)el.feature * rows + irow];
            const bool left = raw_goes_left(v, el.flags, el.threshold,
                                            masks ? masks + (int64_t)el.node * 8 : nullptr,
                                            data_bins);
            const double o = (left == ((el.flags & 0x100u) != 0)) ? 1.0 : 0.0;
#pragma unroll
            for (int u = 0; u < SHAP_MAX_U; ++u)
                if (u == el.uniq) one[u] *= o;
        }
        const int U = P.num_uniq;
        // EXTEND with the dummy element at index 0 (SHAP.swift:266-279)
        double pw[SHAP_MAX_U + 1];
        pw[0] = 1.0;
#pragma unroll
        for (int j = 1; j <= SHAP_MAX_U; ++j) {
            pw[j] = 0.0;
            if (j <= U) {
                const double o = one[j - 1], z = zero[j - 1];
#pragma unroll
                for (int q = j - 1; q >= 0; --q) {
                    pw[q + 1] += o * pw[q] * (double)(q + 1) / (double)(j + 1);
                    pw[q] = z * pw[q] * (double)(j - q) / (double)(j + 1);
                }
            }
        }
        // unwound sums per unique feature (SHAP.swift:307-325)
#pragma unroll
        for (int u = 0; u < SHAP_MAX_U; ++u) {
            if (u < U) {
                const double o = one[u], z = zero[u];
                double total = 0.0;
                if (o != 0.0) {
                    double next = 0.0;
#pragma unroll
                    for (int q = SHAP_MAX_U; q >= 0; --q)
                        if (q == U) next = pw[q];
#pragma unroll
                    for (int q = SHAP_MAX_U - 1; q >= 0; --q) {
                        if (q < U) {
                            const double tmp = next / ((double)(q + 1) * o);
                            total += tmp;
                            next = pw[q] - tmp * z * (double)(U - q);
                        }
                    }
                } else if (z != 0.0) {
#pragma unroll
                    for (int q = SHAP_MAX_U - 1; q >= 0; --q)
                        if (q < U) total += pw[q] / (z * (double)(U - q));
                }
                const double contrib = total * (double)(U + 1) * (o - z) * P.leaf;
                phi[feat[u] * 64 + lane] += contrib;
            }
        }
    }
    if (!valid) return;
    float *orow = out + i * (int64_t)(cols + 1);
    for (int f = 0; f < cols; ++f) orow[f] = (float)phi[f * 64 + lane];
    orow[cols] = bias;
}

// Path-parallel TreeSHAP: one wavefront per row (grid-stride), one lane per
// root-to-leaf path, 64 paths per pass.  The row's feature values and its phi
// sit in LDS; each lane runs the same fp64 EXTEND/UNWIND as k_treeshap for its
// path and adds its unique features' contributions to phi with ds_add_f64.
// One wavefront owns a row's phi, so the order of the adds is fixed (pass
// order, then the LDS unit's lane order) and the output is deterministic.
template <int MAXU>
__global__ __launch_bounds__(64) void k_treeshap_rows(const float *__restrict__ x, int64_t rows,
                                                      int32_t cols, int32_t data_bins,
                                                      const uint32_t *__restrict__ masks,
                                                      const ShapPath *__restrict__ paths,
                                                      int32_t num_paths,
                                                      const ShapElem *__restrict__ elems,
                                                      const ShapUniq *__restrict__ uniq,
                                                      float bias, float *__restrict__ out) {
    extern __shared__ double row_lds[];                // phi [cols], then x [cols] as f32
    double *phi = row_lds;
    float *xr = reinterpret_cast<float *>(row_lds + cols);
    const int lane = threadIdx.x;
    for (int64_t i = blockIdx.x; i < rows; i += gridDim.x) {
        for (int f = lane; f < cols; f += 64) {
            xr[f] = x[(int64_t)f * rows + i];
            phi[f] = 0.0;
        }
        __syncthreads();
        for (int32_t c = 0; c < num_paths; c += 64) {
            const int32_t p = c + lane;
            if (p >= num_paths) continue;
            const ShapPath P = paths[p];
            const int U = P.num_uniq;
            // one[u] is a product of 0/1 indicators: held as bit u of `ones`
            double zero[MAXU];
            int feat[MAXU];
#pragma unroll
            for (int u = 0; u < MAXU; ++u) {
                zero[u] = 1.0;
                feat[u] = 0;
                if (u < U) {
                    const ShapUniq q = uniq[P.uniq_start + u];
                    zero[u] = q.zero;
                    feat[u] = q.feature;
                }
            }
            uint32_t ones = (1u << MAXU) - 1u;
#pragma unroll
            for (int e = 0; e < MAXU; ++e) {
                if (e >= P.num_elem) break;
                const ShapElem el = elems[P.elem_start + e];
                const bool left = raw_goes_left(xr[el.feature], el.flags, el.threshold,
                                                masks ? masks + (int64_t)el.node * 8 : nullptr,
                                                data_bins);
                if (left != ((el.flags & 0x100u) != 0)) ones &= ~(1u << el.uniq);
            }
            double one[MAXU];
#pragma unroll
            for (int u = 0; u < MAXU; ++u) one[u] = ((ones >> u) & 1u) ? 1.0 : 0.0;
            // EXTEND with the dummy element at index 0 (SHAP.swift:266-279).  The
            // weights (q+1)/(j+1) and (j-q)/(j+1) are compile-time constants here,
            // one multiply each instead of a multiply and a divide (a rounding
            // apart from the divided form).
            double pw[MAXU + 1];
            pw[0] = 1.0;
#pragma unroll
            for (int j = 1; j <= MAXU; ++j) {
                pw[j] = 0.0;
                if (j <= U) {
                    const double o = one[j - 1], z = zero[j - 1];
#pragma unroll
                    for (int q = j - 1; q >= 0; --q) {
                        const double up = (double)(q + 1) / (double)(j + 1);
                        const double down = (double)(j - q) / (double)(j + 1);
                        pw[q + 1] += o * pw[q] * up;
                        pw[q] = z * pw[q] * down;
                    }
                }
            }
            // 1 / (U - q) for q < U: U divisions per path, shared by every
            // unique feature's unwinding
            double inv_uq[MAXU];
#pragma unroll
            for (int q = 0; q < MAXU; ++q) inv_uq[q] = q < U ? 1.0 / (double)(U - q) : 0.0;
            // unwound sums per unique feature (SHAP.swift:307-325).  one[u] is 0
            // or 1, so the o != 0 form divides by the constant q + 1 (a multiply
            // by its reciprocal here) and the o == 0 form by z (U - q) (one 1/z
            // per feature).  Both forms share one loop: a wavefront's lanes take
            // both.
#pragma unroll
            for (int u = 0; u < MAXU; ++u) {
                if (u < U) {
                    const double o = one[u], z = zero[u];
                    const bool on = o != 0.0, live = on || z != 0.0;
                    const double inv_z = (!on && z != 0.0) ? 1.0 / z : 0.0;
                    double total = 0.0;
                    double next = 0.0;
#pragma unroll
                    for (int q = MAXU; q >= 0; --q)
                        if (q == U) next = pw[q];
#pragma unroll
                    for (int q = MAXU - 1; q >= 0; --q) {
                        if (q < U) {
                            const double rq = 1.0 / (double)(q + 1);
                            const double tmp = on ? next * rq
                                                  : (live ? pw[q] * inv_z * inv_uq[q] : 0.0);
                            total += tmp;
                            if (on) next = pw[q] - tmp * z * (double)(U - q);
                        }
                    }
                    atomicAdd(&phi[feat[u]], total * (double)(U + 1) * (o - z) * P.leaf);
                }
            }
        }
        __syncthreads();
        float *orow = out + i * (int64_t)(cols + 1);
        for (int f = lane; f < cols; f += 64) orow[f] = (float)phi[f];
        if (lane == 0) orow[cols] = bias;
        __syncthreads();                               // before the next row reuses the LDS
    }
}

// Columns up to which k_treeshap_rows runs (12 B of LDS per column).
constexpr int SHAP_ROW_MAX_COLS = 4096;

bool treeshap_needs_scratch(int cols) { return cols > SHAP_ROW_MAX_COLS; }

hipError_t launch_treeshap(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                           int32_t data_bins, const uint32_t *masks, const ShapPath *paths,
                           int32_t num_paths, int32_t max_elems, const ShapElem *elems,
                           const ShapUniq *uniq, float bias, float *out, double *phi_global) {
    if (rows <= 0) return hipSuccess;
    if (max_elems < 1 || max_elems > SHAP_MAX_U) return hipErrorInvalidValue;
    if (!treeshap_needs_scratch(cols)) {
        // the per-lane path arrays sized to the longest path: fewer registers,
        // more wavefronts per SIMD
        const unsigned blocks = (unsigned)std::min<int64_t>(rows, (int64_t)1 << 22);
        const size_t lds = (size_t)cols * (sizeof(double) + sizeof(float));
#define MBK_SHAP_ROWS(U)                                                                        \
        hipLaunchKernelGGL(k_treeshap_rows<U>, dim3(blocks), dim3(64), lds, s, x, rows, cols,   \
                           data_bins, masks, paths, num_paths, elems, uniq, bias, out)
        if (max_elems <= 4) MBK_SHAP_ROWS(4);
        else if (max_elems <= 6) MBK_SHAP_ROWS(6);
        else if (max_elems <= 8) MBK_SHAP_ROWS(8);
        else MBK_SHAP_ROWS(SHAP_MAX_U);
#undef MBK_SHAP_ROWS
        return hipGetLastError();
    }
    if (!phi_global) return hipErrorInvalidValue;      // wide data: phi in the caller's scratch
    const unsigned blocks = (unsigned)((rows + 63) / 64);
    hipLaunchKernelGGL(k_treeshap, dim3(blocks), dim3(64), 0, s, x, rows, cols, data_bins, masks,
                       paths, num_paths, elems, uniq, bias, out, phi_global);
    return hipGetLastError();
}


}  // namespace mbk
