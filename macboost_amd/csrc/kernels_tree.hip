// kernels_tree.hip — gfx950 kernels of the on-device tree build.
//
// Binning (Shaders.swift:46-76), gradients + maxima (:87-138), quantisation
// (:176-192), histograms (:212-286), sibling subtraction (:313-326), split
// search (:336-464), decisions (:1355-1511) and the row partition
// (:1241-1311), re-designed for CDNA4:
//   * histograms accumulate one packed 64-bit word per (feature, bin) in LDS
//     (quantised gradient sum in the high half, hessian sum in the low half),
//     one ds_add_u64 per (row, feature), and leave exact per-item partials;
//   * the split search runs one 64-lane wavefront per (sibling pair, feature):
//     it reduces the partials, derives the larger sibling by exact integer
//     subtraction and scans all bins with wavefront prefix sums;
//   * the level-wise row partition is a stable two-pass scan, so every node's
//     rows stay in ascending row order and the whole tree is deterministic.
#include "mbk.h"

#include <float.h>
#include <math.h>

namespace mbk {

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float clampf(float x, float lo, float hi) {
    return fminf(fmaxf(x, lo), hi);
}

// exp evaluated in double and rounded to float once; the oracle does the same.
__device__ __forceinline__ float exp_via_double(float x) { return (float)exp((double)x); }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ float f32_from_bits(uint32_t u) { return __uint_as_float(u); }

template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
    const int lane = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        T t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
}

// Lexicographic argmax on (gain desc, seq asc); invalid = (-inf, INT_MAX).
__device__ __forceinline__ void wave_argmax(float &g, int &seq) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float g2 = __shfl_xor(g, o, 64);
        int s2 = __shfl_xor(seq, o, 64);
        if (g2 > g || (g2 == g && s2 < seq)) { g = g2; seq = s2; }
    }
}

__device__ __forceinline__ bool bin_goes_left(uint32_t b, const NodeSplit &s, int32_t nb,
                                              const uint32_t *mask) {
    if (s.flags & FLAG_CATEGORICAL) return (mask[b >> 5] >> (b & 31u)) & 1u;
    if (b == (uint32_t)(nb - 1)) return (s.flags & FLAG_DEFAULT_LEFT) != 0;
    return b <= s.bin;
}

__device__ __forceinline__ float split_gain(float gl, float hl, float gr, float hr, float lambda,
                                            float parent) {
    float a = (gl * gl) / (hl + lambda);
    float b = (gr * gr) / (hr + lambda);
    return (a + b) - parent;
}

// (g, h) of one row for objective `obj` (Shaders.swift:105-135).
__device__ __forceinline__ void row_grad(const GradParams &gp, float f, float y, float w, float &g,
                                         float &h) {
    switch (gp.objective) {
    case 1: {
        float q = 1.0f / (1.0f + exp_via_double(-f));
        float ww = y > 0.5f ? gp.aux : 1.0f;
        g = (q - y) * ww;
        h = fmaxf(q * (1.0f - q), 1e-6f) * ww;
        break;
    }
    case 2: g = f > y ? 1.0f : -1.0f; h = 1.0f; break;
    case 3: g = clampf(f - y, -gp.alpha, gp.alpha); h = 1.0f; break;
    case 4: g = f > y ? (1.0f - gp.alpha) : -gp.alpha; h = 1.0f; break;
    case 5: {
        float mu = exp_via_double(clampf(f, -30.0f, 30.0f));
        g = mu - y; h = fmaxf(mu, 1e-6f);
        break;
    }
    case 6: {
        float fc = clampf(f, -30.0f, 30.0f);
        float e2 = exp_via_double((2.0f - gp.aux) * fc), e1 = exp_via_double((1.0f - gp.aux) * fc);
        g = e2 - y * e1;
        h = fmaxf((2.0f - gp.aux) * e2 - (1.0f - gp.aux) * y * e1, 1e-6f);
        break;
    }
    default: g = f - y; h = 1.0f; break;
    }
    if (gp.has_weights) { g *= w; h *= w; }
}

// ---------------------------------------------------------------------------
// binning: raw f32 -> bin bytes, written to both layouts
// ---------------------------------------------------------------------------

template <int W>
__global__ __launch_bounds__(256) void k_bin_data(const float *__restrict__ x, int64_t rows,
                                                  int32_t cols, int64_t rs, int64_t cs,
                                                  const float *__restrict__ edges,
                                                  const uint8_t *__restrict__ is_cat,
                                                  int32_t nb, uint8_t *__restrict__ tiled,
                                                  uint8_t *__restrict__ fm, int rows_per_block) {
    extern __shared__ float e_lds[];                 // W * (nb - 2)
    const int t = blockIdx.y;
    const int ne = nb - 2;
    const int data_bins = nb - 1;
    const int f0 = t * W;
    const int nf = min(W, cols - f0);
    for (int k = threadIdx.x; k < nf * ne; k += blockDim.x)
        e_lds[k] = edges[(int64_t)f0 * ne + k];
    __syncthreads();
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = min(rows, r0 + rows_per_block);
    for (int64_t i = r0 + threadIdx.x; i < r1; i += blockDim.x) {
        uint32_t words[W / 4];
#pragma unroll
        for (int k = 0; k < W / 4; ++k) words[k] = 0;
#pragma unroll
        for (int k = 0; k < W; ++k) {
            if (k < nf) {
                const int f = f0 + k;
                const float v = x[i * rs + (int64_t)f * cs];
                uint32_t b;
                if (isnan(v)) {
                    b = (uint32_t)data_bins;
                } else if (is_cat[f]) {
                    int c = (int)rintf(v);
                    c = c < 0 ? 0 : (c > data_bins - 1 ? data_bins - 1 : c);
                    b = (uint32_t)c;
                } else {
                    const float *e = e_lds + k * ne;
                    uint32_t lo = 0, hi = (uint32_t)(data_bins - 1);
                    while (lo < hi) {
                        uint32_t mid = (lo + hi) >> 1;
                        if (v > e[mid]) lo = mid + 1; else hi = mid;
                    }
                    b = lo;
                }
                fm[(int64_t)f * rows + i] = (uint8_t)b;
                words[k >> 2] |= b << (8 * (k & 3));
            }
        }
        uint8_t *dst = tiled + ((int64_t)t * rows + i) * W;
        if constexpr (W >= 16) {
#pragma unroll
            for (int k = 0; k < W / 16; ++k)
                reinterpret_cast<uint4 *>(dst)[k] =
                    make_uint4(words[4 * k], words[4 * k + 1], words[4 * k + 2], words[4 * k + 3]);
        } else {
            *reinterpret_cast<uint2 *>(dst) = make_uint2(words[0], words[1]);
        }
    }
}

hipError_t launch_bin_data(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                           int64_t rs, int64_t cs, const float *edges, const uint8_t *is_cat,
                           int32_t nb, int32_t tile_w, int32_t num_tiles, uint8_t *tiled,
                           uint8_t *fm) {
    const int rpb = 4096;
    dim3 grid((unsigned)((rows + rpb - 1) / rpb), (unsigned)num_tiles);
    size_t lds = (size_t)tile_w * (size_t)(nb - 2) * sizeof(float);
    hipError_t e = hipSuccess;
    switch (tile_w) {
    case 8: e = hipFuncSetAttribute((const void *)k_bin_data<8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); break;
    case 16: e = hipFuncSetAttribute((const void *)k_bin_data<16>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); break;
    case 32: e = hipFuncSetAttribute((const void *)k_bin_data<32>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); break;
    case 64: e = hipFuncSetAttribute((const void *)k_bin_data<64>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    switch (tile_w) {
    case 8: hipLaunchKernelGGL(k_bin_data<8>, grid, dim3(256), lds, s, x, rows, cols, rs, cs, edges, is_cat, nb, tiled, fm, rpb); break;
    case 16: hipLaunchKernelGGL(k_bin_data<16>, grid, dim3(256), lds, s, x, rows, cols, rs, cs, edges, is_cat, nb, tiled, fm, rpb); break;
    case 32: hipLaunchKernelGGL(k_bin_data<32>, grid, dim3(256), lds, s, x, rows, cols, rs, cs, edges, is_cat, nb, tiled, fm, rpb); break;
    case 64: hipLaunchKernelGGL(k_bin_data<64>, grid, dim3(256), lds, s, x, rows, cols, rs, cs, edges, is_cat, nb, tiled, fm, rpb); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// per-tree init, gradient maxima, quantisation
// ---------------------------------------------------------------------------

__global__ void k_tree_init(TreeCtl *ctl) {
    uint32_t *w = reinterpret_cast<uint32_t *>(ctl);
    for (int k = threadIdx.x; k < (int)(sizeof(TreeCtl) / 4); k += blockDim.x) w[k] = 0;
}

hipError_t launch_tree_init(hipStream_t s, TreeCtl *ctl) {
    hipLaunchKernelGGL(k_tree_init, dim3(1), dim3(64), 0, s, ctl);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_grad_max(GradParams gp, const float *__restrict__ preds,
                                                  const float *__restrict__ labels,
                                                  const float *__restrict__ weights, int64_t rows,
                                                  TreeCtl *ctl) {
    __shared__ uint32_t red[2][4];
    uint32_t mg = 0, mh = 0;   // max on f32 bit patterns (Shaders.swift:87-94)
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < rows;
         i += (int64_t)gridDim.x * blockDim.x) {
        float g, h;
        row_grad(gp, preds[i], labels[i], gp.has_weights ? weights[i] : 1.0f, g, h);
        mg = max(mg, __float_as_uint(fabsf(g)));
        mh = max(mh, __float_as_uint(h));
    }
    mg = wave_max_u32(mg);
    mh = wave_max_u32(mh);
    const int w = threadIdx.x >> 6;
    if (lane_id() == 0) { red[0][w] = mg; red[1][w] = mh; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t a = red[0][0], b = red[1][0];
        for (int k = 1; k < (int)(blockDim.x >> 6); ++k) { a = max(a, red[0][k]); b = max(b, red[1][k]); }
        atomicMax(&ctl->max_gh[0], a);
        atomicMax(&ctl->max_gh[1], b);
    }
}

hipError_t launch_grad_max(hipStream_t s, const GradParams &gp, const float *preds,
                           const float *labels, const float *weights, int64_t rows,
                           TreeCtl *ctl) {
    int64_t blocks = (rows + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_grad_max, dim3((unsigned)blocks), dim3(256), 0, s, gp, preds, labels,
                       weights, rows, ctl);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_quantize(GradParams gp, const float *__restrict__ preds,
                                                  const float *__restrict__ labels,
                                                  const float *__restrict__ weights, int64_t rows,
                                                  const TreeCtl *ctl, Entry *__restrict__ order) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    const float mg = f32_from_bits(ctl->max_gh[0]), mh = f32_from_bits(ctl->max_gh[1]);
    const float gscale = mg > 0.0f ? 32767.0f / mg : 0.0f;
    const float hscale = mh > 0.0f ? 127.0f / mh : 0.0f;
    float g, h;
    row_grad(gp, preds[i], labels[i], gp.has_weights ? weights[i] : 1.0f, g, h);
    const int qg = (int)rintf(g * gscale);
    const uint32_t qh = (uint32_t)rintf(h * hscale);
    Entry e;
    e.row = (uint32_t)i;
    e.ghq = ((uint32_t)(qg & 0xFFFF) << 16) | (qh & 0x7Fu);
    order[i] = e;
}

hipError_t launch_quantize(hipStream_t s, const GradParams &gp, const float *preds,
                           const float *labels, const float *weights, int64_t rows,
                           const TreeCtl *ctl, Entry *order) {
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, gp,
                       preds, labels, weights, rows, ctl, order);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// histograms: packed 64-bit LDS words, one item per (node chunk, tile)
// ---------------------------------------------------------------------------

template <int W>
__global__ __launch_bounds__(1024) void k_hist(const uint8_t *__restrict__ tiled,
                                               const Entry *__restrict__ order,
                                               const HistItem *__restrict__ items,
                                               const TreeCtl *ctl, uint64_t *__restrict__ partials,
                                               int64_t rows, int32_t cols, int32_t nb) {
    extern __shared__ uint64_t hist_lds[];           // [W][nb]
    constexpr int BYTES = W >= 16 ? 16 : 8;
    constexpr int LPR = W / BYTES;                    // lanes per row
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int words = W * nb;
    const uint32_t nitems = ctl->num_items;
    const int q = tid % LPR;
    const int r0 = tid / LPR;
    const int rstep = nthr / LPR;
    for (uint32_t it = blockIdx.x; it < nitems; it += gridDim.x) {
        const HistItem item = items[it];
        const int nfeat = min(W, cols - (int)item.tile * W);
        for (int k = tid; k < words; k += nthr) hist_lds[k] = 0;
        __syncthreads();
        const uint8_t *tile = tiled + (size_t)item.tile * (size_t)rows * W;
        const Entry *ent = order + item.start;
        for (uint32_t s = r0; s < item.count; s += rstep) {
            const Entry e = ent[s];
            const int32_t qg = (int32_t)(int16_t)(uint16_t)(e.ghq >> 16);
            const uint64_t v = ((uint64_t)(uint32_t)qg << 32) + (uint64_t)(e.ghq & 0x7Fu);
            const uint8_t *p = tile + (size_t)e.row * W + q * BYTES;
            uint32_t wv[BYTES / 4];
            if constexpr (BYTES == 16) {
                const uint4 bb = *reinterpret_cast<const uint4 *>(p);
                wv[0] = bb.x; wv[1] = bb.y; wv[2] = bb.z; wv[3] = bb.w;
            } else {
                const uint2 bb = *reinterpret_cast<const uint2 *>(p);
                wv[0] = bb.x; wv[1] = bb.y;
            }
#pragma unroll
            for (int k = 0; k < BYTES; ++k) {
                const int fl = q * BYTES + k;
                const uint32_t b = (wv[k >> 2] >> (8 * (k & 3))) & 0xFFu;
                if (fl < nfeat && b < (uint32_t)nb) {
                    atomicAdd(reinterpret_cast<unsigned long long *>(&hist_lds[fl * nb + b]),
                              (unsigned long long)v);
                }
            }
        }
        __syncthreads();
        uint64_t *out = partials + (size_t)it * (size_t)words;
        for (int k = tid; k < words; k += nthr) out[k] = hist_lds[k];
        __syncthreads();
    }
}

hipError_t launch_hist(hipStream_t s, const Shape &sh, const uint8_t *tiled, const Entry *order,
                       const HistItem *items, const TreeCtl *ctl, uint64_t *partials, int grid) {
    size_t lds = (size_t)sh.tile_w * (size_t)sh.num_bins * sizeof(uint64_t);
    switch (sh.tile_w) {
#define MBK_HIST_CASE(WW)                                                                        \
    case WW:                                                                                     \
        hipLaunchKernelGGL(k_hist<WW>, dim3(grid), dim3(1024), lds, s, tiled, order, items, ctl, \
                           partials, sh.rows, sh.cols, sh.num_bins);                             \
        break;
        MBK_HIST_CASE(8)
        MBK_HIST_CASE(16)
        MBK_HIST_CASE(32)
        MBK_HIST_CASE(64)
#undef MBK_HIST_CASE
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t hist_set_lds_limit(int tile_w, int num_bins) {
    int bytes = tile_w * num_bins * (int)sizeof(uint64_t);
    hipError_t e = hipSuccess;
    switch (tile_w) {
    case 8: e = hipFuncSetAttribute((const void *)k_hist<8>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); break;
    case 16: e = hipFuncSetAttribute((const void *)k_hist<16>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); break;
    case 32: e = hipFuncSetAttribute((const void *)k_hist<32>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); break;
    case 64: e = hipFuncSetAttribute((const void *)k_hist<64>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); break;
    default: return hipErrorInvalidValue;
    }
    return e;
}

// ---------------------------------------------------------------------------
// split search: one wavefront per (sibling pair, feature)
// ---------------------------------------------------------------------------

struct CatScratch {
    float key[256];
    int64_t sg[256];
    int64_t sh[256];
    uint32_t mask[8];
};

// Best split of one node's feature histogram held as 4 consecutive bins per
// lane (bins 4*lane .. 4*lane+3).  Mirrors find_splits (Shaders.swift:396-463)
// with exact integer prefix sums.  Returns the result in lane 0's `out`.
__device__ void node_split(const int64_t (&hg)[4], const int64_t (&hh)[4], int32_t nb,
                           bool is_cat, int cst, float g_inv, float h_inv, const SplitParams &sp,
                           CatScratch *cs, SplitResult *dst) {
    const int lane = lane_id();
    const int b0 = 4 * lane;
    const int data_bins = nb - 1;
    int64_t lg = 0, lh = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) { lg += hg[j]; lh += hh[j]; }
    const int64_t G_tot = wave_sum(lg), H_tot = wave_sum(lh);
    const float G = (float)G_tot * g_inv, H = (float)H_tot * h_inv;
    const float parent = (G * G) / (H + sp.lambda);

    float best_gain = -INFINITY;
    int best_seq = 0x7FFFFFFF;
    uint32_t best_bin = 0, best_flags = 0;
    float best_gl = 0.0f, best_hl = 0.0f;
    int64_t best_gli = 0, best_hli = 0;

    if (!is_cat) {
        // missing-bin totals live in the lane holding bin nb-1
        const int ml = data_bins >> 2, mj = data_bins & 3;
        int64_t mg = 0, mh = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j == mj) { mg = hg[j]; mh = hh[j]; }
        const int64_t GM = __shfl(mg, ml, 64), HM = __shfl(mh, ml, 64);
        const float Hm = (float)HM * h_inv;
        const int64_t ex_g = wave_inclusive_scan(lg) - lg;
        const int64_t ex_h = wave_inclusive_scan(lh) - lh;
        int64_t GL = ex_g, HL = ex_h;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = b0 + j;
            GL += hg[j];
            HL += hh[j];
            if (b + 1 < data_bins) {
                {   // missing goes right
                    const float gl = (float)GL * g_inv, hl = (float)HL * h_inv;
                    const float gr = (float)(G_tot - GL) * g_inv, hr = (float)(H_tot - HL) * h_inv;
                    if (hl >= sp.min_child_hess && hr >= sp.min_child_hess) {
                        bool ok = true;
                        if (cst != 0) {
                            const float vl = -gl / (hl + sp.lambda), vr = -gr / (hr + sp.lambda);
                            ok = cst > 0 ? vl <= vr : vl >= vr;
                        }
                        const float gain = split_gain(gl, hl, gr, hr, sp.lambda, parent);
                        if (ok && gain > best_gain) {
                            best_gain = gain; best_seq = 2 * b; best_bin = (uint32_t)b;
                            best_flags = 0; best_gl = gl; best_hl = hl; best_gli = GL; best_hli = HL;
                        }
                    }
                }
                if (Hm > 0.0f) {   // missing goes left
                    const int64_t LG = GL + GM, LH = HL + HM;
                    const float lgf = (float)LG * g_inv, lhf = (float)LH * h_inv;
                    const float rg = (float)(G_tot - LG) * g_inv, rh = (float)(H_tot - LH) * h_inv;
                    if (lhf >= sp.min_child_hess && rh >= sp.min_child_hess) {
                        bool ok = true;
                        if (cst != 0) {
                            const float vl = -lgf / (lhf + sp.lambda), vr = -rg / (rh + sp.lambda);
                            ok = cst > 0 ? vl <= vr : vl >= vr;
                        }
                        const float gain = split_gain(lgf, lhf, rg, rh, sp.lambda, parent);
                        if (ok && gain > best_gain) {
                            best_gain = gain; best_seq = 2 * b + 1; best_bin = (uint32_t)b;
                            best_flags = FLAG_DEFAULT_LEFT; best_gl = lgf; best_hl = lhf;
                            best_gli = LG; best_hli = LH;
                        }
                    }
                }
            }
        }
        float wg = best_gain;
        int ws = best_seq;
        wave_argmax(wg, ws);
        if (ws == 0x7FFFFFFF) {
            if (lane == 0) {
                SplitResult r = {};
                r.gain = -INFINITY;
                *dst = r;
            }
        } else if (ws == best_seq && best_gain == wg) {
            SplitResult r = {};
            r.gain = best_gain; r.bin = best_bin; r.gl = best_gl; r.hl = best_hl;
            r.flags = best_flags; r.gl_int = best_gli; r.hl_int = best_hli;
            *dst = r;
        }
        return;
    }

    // Categorical: non-empty bins (missing included) stably sorted by
    // g / (h + catSmooth) (cat_sort, Shaders.swift:339-359), prefixes scanned.
    bool ne[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = b0 + j;
        const float hb = (float)hh[j] * h_inv;
        ne[j] = b < nb && hb > 0.0f;
        cs->key[b] = ne[j] ? ((float)hg[j] * g_inv) / (hb + sp.cat_smooth) : 0.0f;
        cs->sg[b] = 0; cs->sh[b] = 0;
    }
    const uint64_t ne_bits0 = __ballot(ne[0]), ne_bits1 = __ballot(ne[1]);
    const uint64_t ne_bits2 = __ballot(ne[2]), ne_bits3 = __ballot(ne[3]);
    if (lane < 8) cs->mask[lane] = 0;
    __syncthreads();
    const int m = __popcll(ne_bits0) + __popcll(ne_bits1) + __popcll(ne_bits2) + __popcll(ne_bits3);
    int rank[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        rank[j] = -1;
        if (ne[j]) {
            const int b = b0 + j;
            const float kb = cs->key[b];
            int r = 0;
            for (int c = 0; c < nb; ++c) {
                const int cl = c >> 2, cj = c & 3;
                const uint64_t bits = cj == 0 ? ne_bits0 : cj == 1 ? ne_bits1 : cj == 2 ? ne_bits2 : ne_bits3;
                if ((bits >> cl) & 1ull) {
                    const float kc = cs->key[c];
                    r += (kc < kb || (kc == kb && c < b)) ? 1 : 0;
                }
            }
            rank[j] = r;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ne[j]) { cs->sg[rank[j]] = hg[j]; cs->sh[rank[j]] = hh[j]; }
    __syncthreads();
    int64_t pg[4], ph[4];
    int64_t tg = 0, th = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) { pg[j] = cs->sg[b0 + j]; ph[j] = cs->sh[b0 + j]; tg += pg[j]; th += ph[j]; }
    int64_t GL = wave_inclusive_scan(tg) - tg, HL = wave_inclusive_scan(th) - th;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = b0 + j;                         // sorted position
        GL += pg[j];
        HL += ph[j];
        if (i + 1 < m) {
            const float gl = (float)GL * g_inv, hl = (float)HL * h_inv;
            const float gr = (float)(G_tot - GL) * g_inv, hr = (float)(H_tot - HL) * h_inv;
            if (!(hl < sp.min_child_hess || hr < sp.min_child_hess)) {
                const float gain = split_gain(gl, hl, gr, hr, sp.lambda, parent);
                if (gain > best_gain) {
                    best_gain = gain; best_seq = i; best_bin = (uint32_t)(i + 1);
                    best_flags = FLAG_CATEGORICAL; best_gl = gl; best_hl = hl;
                    best_gli = GL; best_hli = HL;
                }
            }
        }
    }
    float wg = best_gain;
    int ws = best_seq;
    wave_argmax(wg, ws);
    if (ws == 0x7FFFFFFF) {
        if (lane == 0) {
            SplitResult r = {};
            r.gain = -INFINITY;
            *dst = r;
        }
        return;
    }
    const int k = ws + 1;                            // left subset size
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ne[j] && rank[j] < k) atomicOr(&cs->mask[(b0 + j) >> 5], 1u << ((b0 + j) & 31));
    __syncthreads();
    if (ws == best_seq && best_gain == wg) {
        SplitResult r = {};
        r.gain = best_gain; r.bin = best_bin; r.gl = best_gl; r.hl = best_hl;
        r.flags = best_flags; r.gl_int = best_gli; r.hl_int = best_hli;
#pragma unroll
        for (int w = 0; w < 8; ++w) r.mask[w] = cs->mask[w];
        *dst = r;
    }
}

__global__ __launch_bounds__(64) void k_split(Shape sh, SplitParams sp,
                                              const Pair *__restrict__ pairs,
                                              const uint64_t *__restrict__ partials,
                                              const int64_t *__restrict__ hist_prev,
                                              int64_t *__restrict__ hist_cur,
                                              const uint8_t *__restrict__ is_cat,
                                              const int8_t *__restrict__ monotone,
                                              const uint8_t *__restrict__ feat_mask,
                                              const TreeCtl *ctl, const uint32_t *count,
                                              int64_t *node_g, int64_t *node_h,
                                              uint32_t level_start,
                                              SplitResult *__restrict__ results) {
    __shared__ CatScratch cs;
    const int F = sh.cols, nb = sh.num_bins, W = sh.tile_w;
    const uint32_t pair_idx = blockIdx.x / (uint32_t)F;
    const int f = (int)(blockIdx.x % (uint32_t)F);
    if (pair_idx >= ctl->num_pairs) return;          // uniform per block (one wave)
    const Pair pr = pairs[pair_idx];
    const int lane = lane_id();
    const int tile = f / W, fl = f % W;
    const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
    const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;

    // built node: reduce its partials for feature f
    int64_t bg[4] = {0, 0, 0, 0}, bh[4] = {0, 0, 0, 0};
    for (uint32_t c = 0; c < pr.nchunks; ++c) {
        const size_t item = (size_t)pr.item_first + (size_t)tile * pr.nchunks + c;
        const uint64_t *src = partials + (item * (size_t)W + (size_t)fl) * (size_t)nb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = 4 * lane + j;
            if (b < nb) {
                const uint64_t w = src[b];
                bg[j] += (int64_t)(int32_t)(uint32_t)(w >> 32);
                bh[j] += (int64_t)(uint32_t)w;
            }
        }
    }
    int64_t *hb = hist_cur + (((size_t)pr.built * F + f) * nb) * 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        if (b < nb) { hb[2 * b] = bg[j]; hb[2 * b + 1] = bh[j]; }
    }
    const bool cat = is_cat[f] != 0;
    const int cst = cat ? 0 : (int)monotone[f];
    const bool allowed = feat_mask[f] != 0;
    const uint32_t nb_abs = level_start + pr.built;
    if (f == 0) {
        const int64_t G = wave_sum(bg[0] + bg[1] + bg[2] + bg[3]);
        const int64_t H = wave_sum(bh[0] + bh[1] + bh[2] + bh[3]);
        if (lane == 0) { node_g[nb_abs] = G; node_h[nb_abs] = H; }
    }
    SplitResult *rb = results + (size_t)pr.built * F + f;
    if (allowed && count[nb_abs] >= 1) {
        node_split(bg, bh, nb, cat, cst, g_inv, h_inv, sp, &cs, rb);
    } else if (lane == 0) {
        SplitResult r = {};
        r.gain = -INFINITY;
        *rb = r;
    }
    if (pr.derived == NONE) return;

    // derived sibling = parent - built (exact), Shaders.swift:313-326
    const int64_t *hp = hist_prev + (((size_t)pr.parent * F + f) * nb) * 2;
    int64_t dg[4], dh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        dg[j] = 0; dh[j] = 0;
        if (b < nb) { dg[j] = hp[2 * b] - bg[j]; dh[j] = hp[2 * b + 1] - bh[j]; }
    }
    int64_t *hd = hist_cur + (((size_t)pr.derived * F + f) * nb) * 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        if (b < nb) { hd[2 * b] = dg[j]; hd[2 * b + 1] = dh[j]; }
    }
    const uint32_t nd_abs = level_start + pr.derived;
    if (f == 0) {
        const int64_t G = wave_sum(dg[0] + dg[1] + dg[2] + dg[3]);
        const int64_t H = wave_sum(dh[0] + dh[1] + dh[2] + dh[3]);
        if (lane == 0) { node_g[nd_abs] = G; node_h[nd_abs] = H; }
    }
    SplitResult *rd = results + (size_t)pr.derived * F + f;
    __syncthreads();
    if (allowed && count[nd_abs] >= 1) {
        node_split(dg, dh, nb, cat, cst, g_inv, h_inv, sp, &cs, rd);
    } else if (lane == 0) {
        SplitResult r = {};
        r.gain = -INFINITY;
        *rd = r;
    }
}

hipError_t launch_split(hipStream_t s, const Shape &sh, const SplitParams &sp, const Pair *pairs,
                        uint32_t max_pairs, const uint64_t *partials, const int64_t *hist_prev,
                        int64_t *hist_cur, const uint8_t *is_cat, const int8_t *monotone,
                        const uint8_t *feat_mask, const TreeCtl *ctl, const uint32_t *count,
                        int64_t *node_g, int64_t *node_h, uint32_t level_start,
                        SplitResult *results) {
    if (sh.num_bins > 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_split, dim3(max_pairs * (uint32_t)sh.cols), dim3(64), 0, s, sh, sp, pairs,
                       partials, hist_prev, hist_cur, is_cat, monotone, feat_mask, ctl, count,
                       node_g, node_h, level_start, results);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decisions: one wavefront per node (decide_splits phase 1, :1386-1451)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(64) void k_decide(Shape sh, SplitParams sp, LevelArgs la,
                                               const SplitResult *__restrict__ results,
                                               const uint32_t *count, int64_t *node_g,
                                               int64_t *node_h, float2 *bounds,
                                               const int8_t *monotone, const TreeCtl *ctl,
                                               uint32_t *left_count, TreeOut out) {
    const uint32_t local = blockIdx.x;
    const uint32_t n = la.level_start + local;
    const int lane = lane_id();
    const int F = sh.cols;
    if (lane == 0) left_count[local] = 0;
    if (count[n] < 1) {
        if (lane == 0) {
            NodeSplit leaf = {-1, 0, 0};
            out.split[n] = leaf;
            out.leaf[n] = 0.0f;
            out.gain[n] = 0.0f;
        }
        return;
    }
    float bg = -INFINITY;
    int bf = 0x7FFFFFFF;
    for (int f = lane; f < F; f += 64) {
        const float g = results[(size_t)local * F + f].gain;
        if (g > bg) { bg = g; bf = f; }               // f ascending within the lane
    }
    wave_argmax(bg, bf);
    if (lane != 0) return;
    const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
    const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;
    const int64_t Gt = node_g[n], Ht = node_h[n];
    if (bf != 0x7FFFFFFF && isfinite(bg) && bg > sp.min_split_gain) {
        const SplitResult r = results[(size_t)local * F + bf];
        NodeSplit ns = {bf, r.bin, r.flags};
        out.split[n] = ns;
        out.leaf[n] = 0.0f;
        out.gain[n] = r.gain;
        const bool cat = (r.flags & FLAG_CATEGORICAL) != 0;
        for (int w = 0; w < 8; ++w) out.mask[(size_t)n * 8 + w] = cat ? r.mask[w] : 0u;
        const uint32_t lc = 2 * n + 1, rc = 2 * n + 2;
        node_g[lc] = r.gl_int; node_h[lc] = r.hl_int;
        node_g[rc] = Gt - r.gl_int; node_h[rc] = Ht - r.hl_int;
        // monotone bounds (Shaders.swift:1424-1443)
        const float2 pb = bounds[n];
        float2 lb = pb, rb = pb;
        const int cst = cat ? 0 : (int)monotone[bf];
        if (cst != 0) {
            const float vl = -r.gl / (r.hl + sp.lambda);
            const float gr = (float)(Gt - r.gl_int) * g_inv, hr = (float)(Ht - r.hl_int) * h_inv;
            const float vr = -gr / (hr + sp.lambda);
            const float mid = clampf(0.5f * (vl + vr), pb.x, pb.y);
            if (cst > 0) { lb.y = fminf(lb.y, mid); rb.x = fmaxf(rb.x, mid); }
            else { lb.x = fmaxf(lb.x, mid); rb.y = fminf(rb.y, mid); }
        }
        bounds[lc] = lb;
        bounds[rc] = rb;
    } else {
        NodeSplit leaf = {-1, 0, 0};
        out.split[n] = leaf;
        out.gain[n] = 0.0f;
        const float2 bb = bounds[n];
        const float G = (float)Gt * g_inv, H = (float)Ht * h_inv;
        out.leaf[n] = sp.learning_rate * clampf(-G / (H + sp.lambda), bb.x, bb.y);
    }
}

hipError_t launch_decide(hipStream_t s, const Shape &sh, const SplitParams &sp,
                         const LevelArgs &la, const SplitResult *results, const uint32_t *count,
                         int64_t *node_g, int64_t *node_h, float2 *bounds,
                         const int8_t *monotone, const TreeCtl *ctl, uint32_t *left_count,
                         TreeOut out) {
    hipLaunchKernelGGL(k_decide, dim3(la.num_level), dim3(64), 0, s, sh, sp, la, results, count,
                       node_g, node_h, bounds, monotone, ctl, left_count, out);
    return hipGetLastError();
}

__global__ void k_final_leaves(SplitParams sp, LevelArgs la, const uint32_t *count,
                               const int64_t *node_g, const int64_t *node_h,
                               const float2 *bounds, const TreeCtl *ctl, TreeOut out) {
    const uint32_t local = blockIdx.x * blockDim.x + threadIdx.x;
    if (local >= la.num_level) return;
    const uint32_t n = la.level_start + local;
    NodeSplit leaf = {-1, 0, 0};
    out.split[n] = leaf;
    out.gain[n] = 0.0f;
    if (count[n] >= 1) {
        const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
        const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;
        const float G = (float)node_g[n] * g_inv, H = (float)node_h[n] * h_inv;
        const float2 bb = bounds[n];
        out.leaf[n] = sp.learning_rate * clampf(-G / (H + sp.lambda), bb.x, bb.y);
    } else {
        out.leaf[n] = 0.0f;
    }
}

hipError_t launch_final_leaves(hipStream_t s, const SplitParams &sp, const LevelArgs &la,
                               const uint32_t *count, const int64_t *node_g,
                               const int64_t *node_h, const float2 *bounds, const TreeCtl *ctl,
                               TreeOut out) {
    hipLaunchKernelGGL(k_final_leaves, dim3((la.num_level + 255) / 256), dim3(256), 0, s, sp, la,
                       count, node_g, node_h, bounds, ctl, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// level planning (single workgroup): segment layout, sibling pairs, items
// ---------------------------------------------------------------------------

// Exclusive scan of v[0..n) in place by one 1024-thread block; returns total.
__device__ uint32_t block_exclusive_scan(uint32_t *v, uint32_t n, uint32_t *wave_tot) {
    const int tid = threadIdx.x;
    const int w = tid >> 6, nw = blockDim.x >> 6;
    uint32_t carry = 0;
    for (uint32_t base = 0; base < n; base += blockDim.x) {
        const uint32_t i = base + tid;
        const uint32_t x = i < n ? v[i] : 0u;
        const uint32_t inc = wave_inclusive_scan(x);
        if (lane_id() == 63) wave_tot[w] = inc;
        __syncthreads();
        if (tid == 0) {
            uint32_t acc = 0;
            for (int k = 0; k < nw; ++k) { uint32_t t = wave_tot[k]; wave_tot[k] = acc; acc += t; }
            wave_tot[nw] = acc;
        }
        __syncthreads();
        if (i < n) v[i] = carry + wave_tot[w] + inc - x;
        carry += wave_tot[nw];
        __syncthreads();
    }
    return carry;
}

__device__ void write_items(const Shape &sh, TreeCtl *ctl, int level, Pair *pairs,
                            HistItem *items, const uint32_t *seg_start,
                            const uint32_t *count_level, uint32_t num_pairs,
                            uint32_t target_items, uint32_t min_chunk, uint32_t *scratch,
                            uint32_t *wave_tot) {
    __shared__ uint32_t s_chunk;
    __shared__ uint32_t s_total;
    const int tid = threadIdx.x;
    // total built rows -> chunk size (accumulated in LDS)
    if (tid == 0) s_total = 0;
    __syncthreads();
    uint32_t part = 0;
    for (uint32_t k = tid; k < num_pairs; k += blockDim.x) part += count_level[pairs[k].built];
    part = wave_sum(part);
    if (lane_id() == 0) atomicAdd(&s_total, part);
    __syncthreads();
    if (tid == 0) {
        const uint64_t total = s_total;
        uint64_t c = (total * (uint64_t)sh.num_tiles + target_items - 1) / (target_items ? target_items : 1);
        if (c < min_chunk) c = min_chunk;
        if (c > HIST_CHUNK_MAX) c = HIST_CHUNK_MAX;
        s_chunk = (uint32_t)c;
        ctl->chunk = (uint32_t)c;
        ctl->level_built[level] = (uint32_t)total;
        scratch[0] = 0;
    }
    __syncthreads();
    const uint32_t chunk = s_chunk;
    // items per pair -> exclusive prefix (scratch[1..num_pairs])
    uint32_t *npair_items = scratch + 1;
    for (uint32_t k = tid; k < num_pairs; k += blockDim.x) {
        const uint32_t c = count_level[pairs[k].built];
        const uint32_t nch = (c + chunk - 1) / chunk;
        pairs[k].nchunks = nch;
        npair_items[k] = nch * (uint32_t)sh.num_tiles;
    }
    __syncthreads();
    const uint32_t total_items = block_exclusive_scan(npair_items, num_pairs, wave_tot);
    for (uint32_t k = tid; k < num_pairs; k += blockDim.x) pairs[k].item_first = npair_items[k];
    if (tid == 0) ctl->num_items = total_items;
    __syncthreads();
    for (uint32_t it = tid; it < total_items; it += blockDim.x) {
        // owning pair: last k with item_first <= it
        uint32_t lo = 0, hi = num_pairs - 1;
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) >> 1;
            if (npair_items[mid] <= it) lo = mid; else hi = mid - 1;
        }
        const Pair pr = pairs[lo];
        const uint32_t rel = it - pr.item_first;
        const uint32_t t = rel / pr.nchunks, c = rel % pr.nchunks;
        const uint32_t cnt = count_level[pr.built];
        HistItem h;
        h.pair = lo;
        h.tile = t;
        h.start = seg_start[pr.built] + c * chunk;
        h.count = min(chunk, cnt - c * chunk);
        items[it] = h;
    }
}

__global__ __launch_bounds__(1024) void k_plan_root(Shape sh, uint32_t rows_active,
                                                    uint32_t target_items, uint32_t min_chunk,
                                                    TreeCtl *ctl, uint32_t *seg_start,
                                                    uint32_t *count, Pair *pairs, HistItem *items,
                                                    float *cover, float2 *bounds, float lo,
                                                    float hi, uint32_t *scratch) {
    __shared__ uint32_t wave_tot[17];
    if (threadIdx.x == 0) {
        count[0] = rows_active;
        seg_start[0] = 0;
        ctl->level_active[0] = rows_active;
        ctl->num_pairs = 1;
        cover[0] = (float)rows_active;
        bounds[0] = make_float2(lo, hi);
        Pair p = {};
        p.built = 0; p.derived = NONE; p.parent = NONE;
        pairs[0] = p;
        scratch[0] = 0;
    }
    __syncthreads();
    write_items(sh, ctl, 0, pairs, items, seg_start, count, 1, target_items, min_chunk, scratch,
                wave_tot);
}

hipError_t launch_plan_root(hipStream_t s, const Shape &sh, uint32_t rows_active,
                            uint32_t target_items, uint32_t min_chunk, TreeCtl *ctl,
                            uint32_t *seg_start, uint32_t *count, Pair *pairs, HistItem *items,
                            float *cover, float2 *bounds, float lo, float hi,
                            uint32_t *scratch) {
    hipLaunchKernelGGL(k_plan_root, dim3(1), dim3(1024), 0, s, sh, rows_active, target_items,
                       min_chunk, ctl, seg_start, count, pairs, items, cover, bounds, lo, hi,
                       scratch);
    return hipGetLastError();
}

// Plan level d from level d-1's routed counts (decide_splits phase 2,
// Shaders.swift:1454-1488, with counts from the partition).
__global__ __launch_bounds__(1024) void k_plan_level(
    Shape sh, LevelArgs la, uint32_t target_items, uint32_t min_chunk, TreeCtl *ctl,
    uint32_t *seg_start_next, uint32_t *count, const uint32_t *left_count,
    uint32_t *node_left_prefix, uint32_t *block_left, const TreeOut out, Pair *pairs,
    HistItem *items, uint32_t *scratch) {
    __shared__ uint32_t wave_tot[17];
    const int tid = threadIdx.x;
    const uint32_t num_prev = la.num_level >> 1;
    const uint32_t ls_prev = (la.level_start - 1) >> 1;   // (2^d - 1 - 1) / 2 = 2^(d-1) - 1
    const uint32_t active_prev = ctl->level_active[la.level - 1];
    const uint32_t nblk = (active_prev + ROUTE_BLOCK - 1) / ROUTE_BLOCK;
    // 1. block offsets for the scatter's global left scan
    block_exclusive_scan(block_left, nblk, wave_tot);
    // 2. per-node exclusive left prefix over level d-1
    for (uint32_t p = tid; p < num_prev; p += blockDim.x) node_left_prefix[p] = left_count[p];
    __syncthreads();
    block_exclusive_scan(node_left_prefix, num_prev, wave_tot);
    // 3. child counts, covers and segment starts
    for (uint32_t p = tid; p < num_prev; p += blockDim.x) {
        const uint32_t n = ls_prev + p;
        const bool split = out.split[n].feature >= 0 && count[n] >= 1;
        const uint32_t cl = split ? left_count[p] : 0u;
        const uint32_t cr = split ? count[n] - left_count[p] : 0u;
        count[la.level_start + 2 * p] = cl;
        count[la.level_start + 2 * p + 1] = cr;
        out.cover[la.level_start + 2 * p] = (float)cl;
        out.cover[la.level_start + 2 * p + 1] = (float)cr;
        seg_start_next[2 * p] = cl + cr;              // scanned below
        seg_start_next[2 * p + 1] = 0;
        scratch[1 + p] = split ? 1u : 0u;
    }
    __syncthreads();
    const uint32_t active = block_exclusive_scan(seg_start_next, la.num_level, wave_tot);
    // even slots now hold the prefix of pair totals; right starts follow the left
    for (uint32_t p = tid; p < num_prev; p += blockDim.x) {
        const uint32_t cl = count[la.level_start + 2 * p];
        seg_start_next[2 * p + 1] = seg_start_next[2 * p] + cl;
    }
    __syncthreads();
    if (tid == 0) ctl->level_active[la.level] = active;
    if (la.terminal) {
        if (tid == 0) { ctl->num_pairs = 0; ctl->num_items = 0; }
        return;
    }
    // 4. sibling pairs for split parents: the smaller child builds, ties go left
    const uint32_t num_pairs = block_exclusive_scan(scratch + 1, num_prev, wave_tot);
    for (uint32_t p = tid; p < num_prev; p += blockDim.x) {
        const uint32_t n = ls_prev + p;
        const bool split = out.split[n].feature >= 0 && count[n] >= 1;
        if (!split) continue;
        const uint32_t cl = count[la.level_start + 2 * p];
        const uint32_t cr = count[la.level_start + 2 * p + 1];
        Pair pr = {};
        pr.built = cl <= cr ? 2 * p : 2 * p + 1;
        pr.derived = cl <= cr ? 2 * p + 1 : 2 * p;
        pr.parent = p;
        pairs[scratch[1 + p]] = pr;
    }
    __syncthreads();
    if (tid == 0) { ctl->num_pairs = num_pairs; scratch[0] = 0; }
    __syncthreads();
    if (num_pairs == 0) {
        if (tid == 0) ctl->num_items = 0;
        return;
    }
    write_items(sh, ctl, la.level, pairs, items, seg_start_next, count + la.level_start,
                num_pairs, target_items, min_chunk, scratch, wave_tot);
}

hipError_t launch_plan_level(hipStream_t s, const Shape &sh, const LevelArgs &la,
                             uint32_t target_items, uint32_t min_chunk, TreeCtl *ctl,
                             uint32_t *seg_start_next, uint32_t *count,
                             const uint32_t *left_count, uint32_t *node_left_prefix,
                             uint32_t *block_left, const TreeOut out, Pair *pairs,
                             HistItem *items, uint32_t *scratch) {
    hipLaunchKernelGGL(k_plan_level, dim3(1), dim3(1024), 0, s, sh, la, target_items, min_chunk,
                       ctl, seg_start_next, count, left_count, node_left_prefix, block_left, out,
                       pairs, items, scratch);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// stable row partition: count pass, then scatter pass (route_samples,
// Shaders.swift:1241-1311, made order-preserving)
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t owner_of(const uint32_t *seg, uint32_t n, uint32_t s) {
    // largest local index with seg[idx] <= s (dead nodes repeat the next start)
    uint32_t lo = 0, hi = n - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        if (seg[mid] <= s) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// dir: 0 = left child, 1 = right child, 2 = node is a leaf
__global__ __launch_bounds__(ROUTE_THREADS) void k_route_count(
    Shape sh, LevelArgs la, const uint8_t *__restrict__ bins_fm, const Entry *__restrict__ order_in,
    const uint32_t *__restrict__ seg_start, const TreeOut out, const TreeCtl *ctl,
    uint8_t *__restrict__ dir, uint32_t *left_count, uint32_t *block_left) {
    extern __shared__ uint32_t rc_lds[];             // seg[num_level], cnt[num_level]
    uint32_t *seg = rc_lds;
    uint32_t *cnt = rc_lds + la.num_level;
    __shared__ uint32_t wsum[ROUTE_THREADS / 64];
    const int tid = threadIdx.x;
    for (uint32_t k = tid; k < la.num_level; k += blockDim.x) { seg[k] = seg_start[k]; cnt[k] = 0; }
    __syncthreads();
    const uint32_t active = ctl->level_active[la.level];
    const uint32_t base = blockIdx.x * ROUTE_BLOCK + tid * ROUTE_PER_THREAD;
    uint32_t lefts = 0;
    uint32_t run_node = 0xFFFFFFFFu, run_cnt = 0;   // this thread's entries are contiguous
    uint8_t d8[ROUTE_PER_THREAD];
#pragma unroll
    for (int k = 0; k < ROUTE_PER_THREAD; ++k) {
        const uint32_t s = base + k;
        d8[k] = 2;
        if (s < active) {
            const uint32_t local = owner_of(seg, la.num_level, s);
            const uint32_t n = la.level_start + local;
            const NodeSplit sp = out.split[n];
            if (sp.feature >= 0) {
                const uint32_t row = order_in[s].row;
                const uint32_t b = bins_fm[(size_t)sp.feature * (size_t)sh.rows + row];
                const bool left = bin_goes_left(b, sp, sh.num_bins, out.mask + (size_t)n * 8);
                d8[k] = left ? 0 : 1;
                if (left) {
                    ++lefts;
                    if (local != run_node) {
                        if (run_cnt) atomicAdd(&cnt[run_node], run_cnt);
                        run_node = local;
                        run_cnt = 0;
                    }
                    ++run_cnt;
                }
            }
        }
    }
    if (run_cnt) atomicAdd(&cnt[run_node], run_cnt);
    if (base < active) {
        if (base + ROUTE_PER_THREAD <= active) {
            uint2 packed;
            packed.x = d8[0] | (d8[1] << 8) | (d8[2] << 16) | ((uint32_t)d8[3] << 24);
            packed.y = d8[4] | (d8[5] << 8) | (d8[6] << 16) | ((uint32_t)d8[7] << 24);
            *reinterpret_cast<uint2 *>(dir + base) = packed;
        } else {
            for (int k = 0; k < ROUTE_PER_THREAD; ++k)
                if (base + k < active) dir[base + k] = d8[k];
        }
    }
    lefts = wave_sum(lefts);
    if (lane_id() == 0) wsum[tid >> 6] = lefts;
    __syncthreads();
    if (tid == 0) {
        uint32_t t = 0;
        for (int k = 0; k < ROUTE_THREADS / 64; ++k) t += wsum[k];
        block_left[blockIdx.x] = t;
    }
    for (uint32_t k = tid; k < la.num_level; k += blockDim.x)
        if (cnt[k]) atomicAdd(&left_count[k], cnt[k]);
}

hipError_t launch_route_count(hipStream_t s, const Shape &sh, const LevelArgs &la,
                              const uint8_t *bins_fm, const Entry *order_in,
                              const uint32_t *seg_start, const TreeOut out, const TreeCtl *ctl,
                              uint8_t *dir, uint32_t *left_count, uint32_t *block_left,
                              uint32_t max_blocks) {
    size_t lds = 2 * (size_t)la.num_level * sizeof(uint32_t);
    hipLaunchKernelGGL(k_route_count, dim3(max_blocks), dim3(ROUTE_THREADS), lds, s, sh, la,
                       bins_fm, order_in, seg_start, out, ctl, dir, left_count, block_left);
    return hipGetLastError();
}

__global__ __launch_bounds__(ROUTE_THREADS) void k_route_scatter(
    Shape sh, LevelArgs la, const Entry *__restrict__ order_in, Entry *__restrict__ order_out,
    const uint8_t *__restrict__ dir, const uint32_t *__restrict__ seg_start,
    const uint32_t *__restrict__ seg_start_next, const uint32_t *__restrict__ node_left_prefix,
    const uint32_t *__restrict__ block_off, const TreeOut out, const TreeCtl *ctl,
    float *__restrict__ preds) {
    extern __shared__ uint32_t rs_lds[];             // seg[num_level]
    __shared__ uint32_t wsum[ROUTE_THREADS / 64 + 1];
    uint32_t *seg = rs_lds;
    const int tid = threadIdx.x;
    for (uint32_t k = tid; k < la.num_level; k += blockDim.x) seg[k] = seg_start[k];
    const uint32_t active = ctl->level_active[la.level];
    const uint32_t base = blockIdx.x * ROUTE_BLOCK + tid * ROUTE_PER_THREAD;
    uint8_t d8[ROUTE_PER_THREAD];
    uint32_t lefts = 0;
#pragma unroll
    for (int k = 0; k < ROUTE_PER_THREAD; ++k) {
        const uint32_t s = base + k;
        d8[k] = s < active ? dir[s] : 3;
        lefts += d8[k] == 0 ? 1u : 0u;
    }
    // block exclusive scan of per-thread left counts
    const uint32_t inc = wave_inclusive_scan(lefts);
    if (lane_id() == 63) wsum[tid >> 6] = inc;
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        for (int k = 0; k < ROUTE_THREADS / 64; ++k) { uint32_t t = wsum[k]; wsum[k] = acc; acc += t; }
    }
    __syncthreads();
    uint32_t scan_l = block_off[blockIdx.x] + wsum[tid >> 6] + inc - lefts;
#pragma unroll
    for (int k = 0; k < ROUTE_PER_THREAD; ++k) {
        const uint32_t s = base + k;
        if (d8[k] > 2) continue;
        const uint32_t local = owner_of(seg, la.num_level, s);
        const uint32_t n = la.level_start + local;
        const Entry e = order_in[s];
        if (d8[k] == 2) {
            preds[e.row] += out.leaf[n];
        } else if (la.terminal) {
            preds[e.row] += out.leaf[2 * n + 1 + d8[k]];
        } else {
            const uint32_t lrank = scan_l - node_left_prefix[local];
            uint32_t pos;
            if (d8[k] == 0) pos = seg_start_next[2 * local] + lrank;
            else pos = seg_start_next[2 * local + 1] + (s - seg[local]) - lrank;
            order_out[pos] = e;
        }
        if (d8[k] == 0) ++scan_l;
    }
}

hipError_t launch_route_scatter(hipStream_t s, const Shape &sh, const LevelArgs &la,
                                const Entry *order_in, Entry *order_out, const uint8_t *dir,
                                const uint32_t *seg_start, const uint32_t *seg_start_next,
                                const uint32_t *node_left_prefix, const uint32_t *block_off,
                                const TreeOut out, const TreeCtl *ctl, float *preds,
                                uint32_t max_blocks) {
    size_t lds = (size_t)la.num_level * sizeof(uint32_t);
    hipLaunchKernelGGL(k_route_scatter, dim3(max_blocks), dim3(ROUTE_THREADS), lds, s, sh, la,
                       order_in, order_out, dir, seg_start, seg_start_next, node_left_prefix,
                       block_off, out, ctl, preds);
    return hipGetLastError();
}

}  // namespace mbk
