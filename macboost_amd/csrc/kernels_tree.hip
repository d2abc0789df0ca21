// kernels_tree.hip — gfx950 kernels of the on-device tree build.
//
// Binning (Shaders.swift:46-76), gradients + maxima (:87-138), quantisation
// (:176-192), histograms (:212-286), sibling subtraction (:313-326), split
// search (:336-464), decisions (:1355-1511) and the row partition
// (:1241-1311), re-designed for CDNA4:
//   * histograms accumulate one packed 64-bit word per (feature, bin) in LDS
//     (quantised gradient sum above bit 27, hessian sum below), one
//     ds_add_u64 per (row, feature), and leave exact per-item partials;
//   * partials are reduced into exact int64 histograms, the larger sibling is
//     derived by integer subtraction, and the split search runs one 64-lane
//     wavefront per (sibling pair, feature) with wavefront prefix sums;
//   * the level-wise row partition is one pass that splits every node's
//     interval in place between its children; nothing downstream depends on
//     the order of rows inside a node, so the tree is deterministic.
#include <hip/hip_ext.h>

#include "grad.h"
#include "mbk.h"

#include <float.h>
#include <math.h>
#include <type_traits>

namespace mbk {

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ float f32_from_bits(uint32_t u) { return __uint_as_float(u); }

// One DPP move of a 32- or 64-bit value (64-bit: both halves with the same
// control); lanes without a source, or outside row_mask / bank_mask, get 0.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ uint32_t dpp_move(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ uint64_t dpp_move(uint64_t v) {
    const uint32_t lo = dpp_move<CTRL, ROW_MASK, BANK_MASK>((uint32_t)v);
    const uint32_t hi = dpp_move<CTRL, ROW_MASK, BANK_MASK>((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Inclusive wavefront prefix sum of integers with DPP: row_shr 1, 2, 4, 8
// scan each row of 16 lanes (Hillis-Steele; a lane without a source adds 0),
// then row_bcast:15 adds row 0's total to row 1 and row 2's to row 3, and
// row_bcast:31 adds lane 31's to rows 2 and 3.  Six steps, no LDS round trip
// (a __shfl_up scan is six ds_bpermute round trips).  Integer addition, so
// the result is the exact prefix sum whatever the order.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit integers");
    using U = typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type;
    U u = (U)v;
    u += dpp_move<0x111, 0xf, 0xf>(u);               // row_shr:1
    u += dpp_move<0x112, 0xf, 0xf>(u);               // row_shr:2
    u += dpp_move<0x114, 0xf, 0xf>(u);               // row_shr:4
    u += dpp_move<0x118, 0xf, 0xf>(u);               // row_shr:8
    u += dpp_move<0x142, 0xa, 0xf>(u);               // row_bcast:15 into rows 1 and 3
    u += dpp_move<0x143, 0xc, 0xf>(u);               // row_bcast:31 into rows 2 and 3
    return (T)u;
}

// Lane 63's value in every lane (two readlanes for 64 bits).
template <typename T>
__device__ __forceinline__ T wave_last(T v) {
    if constexpr (sizeof(T) == 8) {
        const uint64_t u = (uint64_t)v;
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
        return (T)(((uint64_t)hi << 32) | lo);
    } else {
        return (T)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    }
}

// Wavefront totals in every lane, from the DPP scan's lane 63 (integer sums
// and maxima: exact in any order).  Every lane of the wavefront must be active.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    static_assert(std::is_integral<T>::value, "integer sums only");
    return wave_last(wave_inclusive_scan(v));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    // lanes without a source read 0, the identity of an unsigned max
    v = max(v, dpp_move<0x111, 0xf, 0xf>(v));        // row_shr:1
    v = max(v, dpp_move<0x112, 0xf, 0xf>(v));        // row_shr:2
    v = max(v, dpp_move<0x114, 0xf, 0xf>(v));        // row_shr:4
    v = max(v, dpp_move<0x118, 0xf, 0xf>(v));        // row_shr:8
    v = max(v, dpp_move<0x142, 0xa, 0xf>(v));        // row_bcast:15
    v = max(v, dpp_move<0x143, 0xc, 0xf>(v));        // row_bcast:31
    return wave_last(v);
}

// Set bits of mask in the lanes below this one.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
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

// (g, h) of row i, multiclass included: the softmax gradient of class
// gp.class_index over preds [K][rows] (compute_gradients_multiclass,
// Shaders.swift:145-170; each exp in double, rounded once).
__device__ __forceinline__ void row_grad_at(const GradParams &gp, const float *__restrict__ preds,
                                            const float *__restrict__ labels,
                                            const float *__restrict__ weights, int64_t i,
                                            float &g, float &h) {
    const float w = gp.has_weights ? weights[i] : 1.0f;
    if (gp.objective != 7) {
        // streamed once per pass, nontemporal (measured: ~1% per tree)
        row_grad(gp, __builtin_nontemporal_load(&preds[i]), __builtin_nontemporal_load(&labels[i]),
                 w, g, h);
        return;
    }
    float m = -INFINITY;
    for (int k = 0; k < gp.num_classes; ++k) m = fmaxf(m, preds[(int64_t)k * gp.rows + i]);
    float sum = 0.0f;
    for (int k = 0; k < gp.num_classes; ++k)
        sum += exp_via_double(preds[(int64_t)k * gp.rows + i] - m);
    const float pk = exp_via_double(preds[(int64_t)gp.class_index * gp.rows + i] - m) / sum;
    const float yk = (int32_t)labels[i] == gp.class_index ? 1.0f : 0.0f;
    g = pk - yk;
    h = fmaxf(2.0f * pk * (1.0f - pk), 1e-6f);
    if (gp.has_weights) { g *= w; h *= w; }
}

// ---------------------------------------------------------------------------
// binning (bin_data, Shaders.swift:46-76): raw f32 -> bin bytes, written to
// both layouts: the gather layout [rows][T][W] (row r's tile t at
// (r*T + t)*W) and the feature-major [F][rows].
//
// A block bins one whole tile (W features) of BIN_ROWS rows, one row per
// thread, 16 features at a time: every row's W-byte tile segment is written
// by one block, the T blocks of a row block run on one XCD (the pieces of a
// row meet in one L2; pieces from blocks on different XCDs went to HBM as
// partial lines), and the feature-major bytes go out as
// one byte per lane, 64 consecutive bytes per wavefront store.  A value's bin
// is the number of edges below it, lower_bound(edges, v) for the
// non-decreasing quantile edges (the reference's binary search).  Each
// feature's edges sit in LDS as the perfect 4-ary search tree over the 256
// bins (255 keys, +inf padded) in breadth-first order, three keys per node:
// four dependent steps of three independent LDS reads and compares (where a
// binary tree needs eight dependent reads), each level's nodes contiguous so
// the lanes of a wavefront spread over the banks; the final node's index in
// the leaf level is the bin.  Tiles past the last feature write zero bytes, so the
// gather layout needs no clearing.
// ---------------------------------------------------------------------------

constexpr int BIN_THREADS = 1024;
constexpr int BIN_ROWS = 4096;                        // rows per block

template <int W>
__global__ __launch_bounds__(BIN_THREADS) void k_bin_data(
    const float *__restrict__ x, int64_t rows, int32_t cols, int64_t rs, int64_t cs,
    const float *__restrict__ edges, const uint8_t *__restrict__ is_cat, int32_t nb, int32_t T,
    int32_t t_first, int32_t t_count, uint8_t *__restrict__ tiled, uint8_t *__restrict__ fm,
    int vec_rows) {
    constexpr int G = W < 16 ? W : 16;               // features per pass
    __shared__ float e_lds[W * 256];                 // [feature][BFS slot 1..255], slot 0 unused
    const int tid = threadIdx.x;
    const int ne = nb - 2, data_bins = nb - 1;
    // Workgroups go to the 8 XCDs round-robin (block b to XCD b % 8): the
    // tiles t_first .. t_first + t_count - 1 of a row block are blocks
    // xcd + 8 (q t_count + t), all on one XCD, so the pieces of a row's bytes
    // merge in that XCD's L2.
    const uint32_t xcd = blockIdx.x & 7u, k8 = blockIdx.x >> 3;
    const int t = t_first + (int)(k8 % (uint32_t)t_count);
    const int64_t row_block = (int64_t)(k8 / (uint32_t)t_count) * 8 + xcd;
    if (row_block * BIN_ROWS >= rows) return;         // grid padding (whole block)
    const int f0 = t * W;
    const int nf = max(0, min(W, cols - f0));         // real features of the tile
    for (int k = tid; k < W * 256; k += BIN_THREADS) {
        const int f = k >> 8, i = k & 255;
        float val = INFINITY;
        if (i < 255 && f < nf) {
            // slot i is key kk (1..3) of node n = i / 3 of the perfect 4-ary
            // tree over the 256 bins in breadth-first order: node n at depth L,
            // position q in its level, splits its span of s = 256 / 4^L bins
            // at q s + kk s / 4, i.e. holds sorted edge q s + kk s / 4 - 1
            const int n = i / 3, kk = i - 3 * n + 1;
            const int L = n == 0 ? 0 : n < 5 ? 1 : n < 21 ? 2 : 3;
            const int q = n - ((1 << (2 * L)) - 1) / 3, span = 256 >> (2 * L);
            const int j = q * span + kk * (span >> 2) - 1;
            if (j < ne) val = edges[(int64_t)(f0 + f) * ne + j];
        }
        e_lds[k] = val;
    }
    uint64_t cat_bits = 0;
    for (int k = 0; k < nf; ++k) cat_bits |= (uint64_t)(is_cat[f0 + k] ? 1u : 0u) << k;
    __syncthreads();
    const int64_t blk0 = row_block * BIN_ROWS;
    const int64_t blk1 = min(rows, blk0 + BIN_ROWS);
    // G values of row r from feature f0 + c on (row-major input 16-B
    // aligned: 16-B loads)
    auto load = [&](int64_t r, int c, float (&v)[G]) {
        const int fc = f0 + c;
        if (vec_rows != 0 && (fc & 3) == 0 && c + G <= nf) {
            const float4 *src = reinterpret_cast<const float4 *>(x + r * rs + fc);
#pragma unroll
            for (int q = 0; q < G / 4; ++q) {
                const float4 w4 = src[q];
                v[4 * q] = w4.x; v[4 * q + 1] = w4.y; v[4 * q + 2] = w4.z; v[4 * q + 3] = w4.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < G; ++k)
                v[k] = c + k < nf ? x[r * rs + (int64_t)(fc + k) * cs] : 0.0f;
        }
    };
    for (int64_t r = blk0 + tid; r < blk1; r += BIN_THREADS) {
        // the row's W tile bytes: each pass shifts its G bytes in at the end,
        // so after the W / G passes they are in order (fixed register indexes
        // in a loop the compiler keeps rolled)
        uint32_t seg[W / 4];
        auto shift_in = [&](const uint32_t (&w4)[G / 4]) {
#pragma unroll
            for (int q = 0; q + G / 4 < W / 4; ++q) seg[q] = seg[q + G / 4];
#pragma unroll
            for (int q = 0; q < G / 4; ++q) seg[W / 4 - G / 4 + q] = w4[q];
        };
#pragma unroll 1
        for (int c = 0; c < W; c += G) {
            if (c >= nf) {                            // a last tile's padding: zeros, no search
                const uint32_t zero[G / 4] = {};
                shift_in(zero);
                continue;
            }
            float v[G];
            load(r, c, v);
            uint32_t b[G];
#pragma unroll
            for (int k0 = 0; k0 < G; k0 += 4) {
                if (c + k0 >= nf) {                   // padding features of this pass
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[k0 + j] = 0u;
                    continue;
                }
                // four levels of three comparisons: the child 4 n + 1 + (keys
                // below v); the leaf's index in its level is the bin
                uint32_t ix[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) ix[j] = 0;
#pragma unroll
                for (int level = 0; level < 4; ++level) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float *nk = e_lds + (c + k0 + j) * 256 + 3 * (int)ix[j];
                        const float x = v[k0 + j];
                        ix[j] = 4 * ix[j] + 1 + (x > nk[0] ? 1u : 0u) + (x > nk[1] ? 1u : 0u) +
                                (x > nk[2] ? 1u : 0u);
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = k0 + j;
                    const float val = v[k];
                    uint32_t bb = ix[j] - 85u;               // 85 = (4^4 - 1) / 3
                    if (isnan(val)) {
                        bb = (uint32_t)data_bins;
                    } else if ((cat_bits >> (c + k)) & 1u) {
                        int cc = (int)rintf(val);
                        cc = cc < 0 ? 0 : (cc > data_bins - 1 ? data_bins - 1 : cc);
                        bb = (uint32_t)cc;
                    }
                    b[k] = c + k < nf ? bb : 0u;
                }
            }
            uint32_t w4[G / 4];
#pragma unroll
            for (int q = 0; q < G / 4; ++q)
                w4[q] = b[4 * q] | (b[4 * q + 1] << 8) | (b[4 * q + 2] << 16) | (b[4 * q + 3] << 24);
            shift_in(w4);
#pragma unroll
            for (int k = 0; k < G; ++k)
                if (c + k < nf) fm[(int64_t)(f0 + c + k) * rows + r] = (uint8_t)b[k];
        }
        // the whole segment in back-to-back stores: a 64-B segment reaches L2
        // complete (16-B pieces stored a search apart were written back
        // piecewise, as partial HBM writes)
        uint8_t *dst = tiled + (r * T + t) * (int64_t)W;
        if constexpr (W >= 16) {
#pragma unroll
            for (int q = 0; q < W / 16; ++q)
                reinterpret_cast<uint4 *>(dst)[q] =
                    make_uint4(seg[4 * q], seg[4 * q + 1], seg[4 * q + 2], seg[4 * q + 3]);
        } else {
            *reinterpret_cast<uint2 *>(dst) = make_uint2(seg[0], seg[1]);
        }
    }
}

hipError_t launch_bin_data(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                           int64_t rs, int64_t cs, const float *edges, const uint8_t *is_cat,
                           int32_t nb, int32_t tile_w, int32_t num_tiles, uint8_t *tiled,
                           uint8_t *fm) {
    return launch_bin_tiles(s, x, rows, cols, rs, cs, edges, is_cat, nb, tile_w, num_tiles, 0,
                            num_tiles, tiled, fm);
}

hipError_t launch_bin_tiles(hipStream_t s, const float *x, int64_t rows, int32_t cols,
                            int64_t rs, int64_t cs, const float *edges, const uint8_t *is_cat,
                            int32_t nb, int32_t tile_w, int32_t num_tiles, int32_t tile_first,
                            int32_t tile_count, uint8_t *tiled, uint8_t *fm) {
    if (nb < 4 || nb > 256 || rows <= 0) return rows == 0 ? hipSuccess : hipErrorInvalidValue;
    if (tile_w != 8 && tile_w != 16 && tile_w != 32 && tile_w != 64) return hipErrorInvalidValue;
    if (num_tiles < 1 || (int64_t)num_tiles * tile_w < cols) return hipErrorInvalidValue;
    if (tile_first < 0 || tile_count < 1 || tile_first + tile_count > num_tiles)
        return hipErrorInvalidValue;
    const int64_t nblk = ((rows + BIN_ROWS - 1) / BIN_ROWS + 7) / 8 * 8 * (int64_t)tile_count;
    if (nblk > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nblk);
    const int vec_rows = cs == 1 && (rs & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
#define MBK_BIN(WW)                                                                             \
    hipLaunchKernelGGL(k_bin_data<WW>, grid, dim3(BIN_THREADS), 0, s, x, rows, cols, rs, cs, edges, \
                       is_cat, nb, num_tiles, tile_first, tile_count, tiled, fm, vec_rows)
    if (tile_w == 64) MBK_BIN(64);
    else if (tile_w == 32) MBK_BIN(32);
    else if (tile_w == 16) MBK_BIN(16);
    else MBK_BIN(8);
#undef MBK_BIN
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// the .mbds bin layout (Dataset.swift:18, bin_index, Shaders.swift:37-39):
// 8-feature groups, feature 8g + j of row r at byte (g*rows + r)*8 + j.
// One thread per (row, group) moves one 8-byte word.
// ---------------------------------------------------------------------------

__global__ void k_fm_to_tile8(const uint8_t *__restrict__ fm, int64_t rows, int32_t cols,
                              uint64_t *__restrict__ out) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int g = blockIdx.y;
    if (r >= rows) return;
    uint64_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int f = 8 * g + j;
        if (f < cols) v |= (uint64_t)fm[(int64_t)f * rows + r] << (8 * j);
    }
    out[(int64_t)g * rows + r] = v;
}

// Tile-8 words -> gather layout [rows][T][W] (W a multiple of 8, pre-zeroed)
// and feature-major [F][rows]; pad bytes past the last feature become 0 and
// a bin >= nb raises *bad.
__global__ void k_tile8_to_layouts(const uint64_t *__restrict__ in, int64_t rows, int32_t cols,
                                   int32_t nb, int32_t W, int32_t T, uint8_t *__restrict__ tiled,
                                   uint8_t *__restrict__ fm, uint32_t *bad) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int g = blockIdx.y;
    if (r >= rows) return;
    uint64_t v = in[(int64_t)g * rows + r];
    const int nf = min(8, cols - 8 * g);
    if (nf < 8) v &= (1ull << (8 * nf)) - 1ull;
    bool over = false;
    for (int j = 0; j < nf; ++j) {
        const uint32_t b = (uint32_t)(v >> (8 * j)) & 0xFFu;
        fm[(int64_t)(8 * g + j) * rows + r] = (uint8_t)b;
        over = over || b >= (uint32_t)nb;
    }
    const int f0 = 8 * g, t = f0 / W, c0 = f0 % W;
    *reinterpret_cast<uint64_t *>(tiled + ((size_t)r * (size_t)T + (size_t)t) * (size_t)W + c0) = v;
    if (over) atomicOr(bad, 1u);
}

// ---------------------------------------------------------------------------
// Checks of device-resident raw features (the host path reads host memory):
// a strided row sample for the leakage check, and the categorical id rule of
// Booster.swift:1810-1826.
// ---------------------------------------------------------------------------

// out[k * cols + f] = x[(k * step) * rs + f * cs] for k < m.
__global__ __launch_bounds__(256) void k_gather_sample(const float *__restrict__ x, int64_t rs,
                                                       int64_t cs, int64_t step, int64_t m,
                                                       int32_t cols, float *__restrict__ out) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= m * cols) return;
    const int64_t k = j / cols;
    const int64_t f = j - k * cols;
    out[j] = x[k * step * rs + f * cs];
}

hipError_t launch_gather_sample(hipStream_t s, const float *x, int64_t rs, int64_t cs,
                                int64_t step, int64_t m, int32_t cols, float *out) {
    const int64_t n = m * cols;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_gather_sample, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, rs,
                       cs, step, m, cols, out);
    return hipGetLastError();
}

// Column cat_cols[j] must hold NaN or an integer id in [0, data_bins):
// first_bad[j] (all ones on entry) becomes the first row that does not.
__global__ __launch_bounds__(256) void k_check_categorical(const float *__restrict__ x,
                                                           int64_t rows, int64_t rs, int64_t cs,
                                                           const int32_t *__restrict__ cat_cols,
                                                           int32_t data_bins,
                                                           uint32_t *first_bad) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows) return;
    const float v = x[i * rs + (int64_t)cat_cols[blockIdx.y] * cs];
    if (isnan(v)) return;
    const float c = rintf(v);
    if (!(c >= 0.0f) || !isfinite(c) || c >= (float)data_bins)
        atomicMin(&first_bad[blockIdx.y], (uint32_t)i);
}

hipError_t launch_check_categorical(hipStream_t s, const float *x, int64_t rows, int64_t rs,
                                    int64_t cs, const int32_t *cat_cols, int32_t ncat,
                                    int32_t data_bins, uint32_t *first_bad) {
    if (rows <= 0 || ncat <= 0) return hipSuccess;
    if (ncat > 65535 || (rows + 255) / 256 > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_check_categorical, dim3((unsigned)((rows + 255) / 256), (unsigned)ncat),
                       dim3(256), 0, s, x, rows, rs, cs, cat_cols, data_bins, first_bad);
    return hipGetLastError();
}

hipError_t launch_fm_to_tile8(hipStream_t s, const uint8_t *fm, int64_t rows, int32_t cols,
                              uint64_t *out) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 255) / 256), (unsigned)((cols + 7) / 8));
    hipLaunchKernelGGL(k_fm_to_tile8, grid, dim3(256), 0, s, fm, rows, cols, out);
    return hipGetLastError();
}

hipError_t launch_tile8_to_layouts(hipStream_t s, const uint64_t *in, int64_t rows, int32_t cols,
                                   int32_t nb, int32_t W, int32_t T, uint8_t *tiled, uint8_t *fm,
                                   uint32_t *bad) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (W % 8 != 0 || (int64_t)T * W < cols) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 255) / 256), (unsigned)((cols + 7) / 8));
    hipLaunchKernelGGL(k_tile8_to_layouts, grid, dim3(256), 0, s, in, rows, cols, nb, W, T, tiled,
                       fm, bad);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// quantile edges on the device (Binner.swift:25-56): per feature, the stride
// subsample of non-NaN values, sorted, edge k = sample[min(m-1, (k+1)*m/dataBins)].
// The sample becomes order-preserving u32 keys (one thread per sample), a
// stable LSD radix sort over position chunks of each column orders them
// (4-bit digits, count and scatter launches per pass) and the edges are read
// at their ranks.
// ---------------------------------------------------------------------------

constexpr int EDGE_THREADS = 1024;
constexpr int EDGE_WAVES = EDGE_THREADS / 64;

__device__ __forceinline__ uint32_t float_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wavefront max of unsigned values: DPP row shifts, then row broadcasts
// (lane 63 holds the maximum), read back into every lane.
__device__ __forceinline__ uint32_t wave_max_dpp(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x113, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xe, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xc, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// What a pick of node n needs: bit 0 expanded, bit 1 both children hold
// rows; the children's candidate gains as ordered keys (0: none).
struct LWBInfo {
    uint32_t flags, kl, kr, pad;
};
// Order key of a gain (+0 and -0 alike, as the float comparisons see them).
__device__ __forceinline__ uint32_t gain_key(float g) { return float_key(g == 0.0f ? 0.0f : g); }
constexpr int LWB_EVAL = 4;   // nodes one wavefront evaluates at once

// Open-mask words (one bit per candidate rank) for a tree of depth D.
constexpr int lwb_mask_words(int depth) { return ((1 << (depth + 1)) - 1 + 63) / 64; }

// Register slots per lane of the repeated-gain replay: an open list of up to
// 2 * LWB_MAX_LEAVES entries.
constexpr int LWB_SLOTS = (2 * LWB_MAX_LEAVES + 2 + 63) / 64;

__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

constexpr int KEY_STRIDE = SPLIT_KEY_STRIDE;

// A node's split-search key: the ordered gain of one feature's best split
// above, the complement of the feature below, so the 64-bit maximum over the
// node's features is decide_splits' argmax (Shaders.swift:1386-1400): the
// largest gain, the lowest feature among equal gains.  0 is no candidate:
// NaN and -inf gains never win that argmax.
__device__ __forceinline__ uint64_t split_key(float gain, int f) {
    if (!(gain > -INFINITY)) return 0;
    return ((uint64_t)gain_key(gain) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)f);
}
__device__ __forceinline__ int key_feature(uint64_t k) {
    return k ? (int)(0xFFFFFFFFu - (uint32_t)k) : -1;
}
// Whether a node of cnt rows splits: decide_node's test on its key.
__device__ __forceinline__ bool key_splits(uint64_t k, uint32_t cnt, float min_split_gain) {
    if (k == 0 || cnt < 1) return false;
    const float g = key_float((uint32_t)(k >> 32));
    return isfinite(g) && g > min_split_gain;
}

// Sample keys: thread s converts sample s (row s * step) of column blockIdx.y
// into its order-preserving key, NaN into 0xFFFFFFFF (above every number's
// key, so NaNs sort last and the first m sorted keys are the sample's m
// non-NaN values).  Categorical columns take no sample.
constexpr int EDGE_SAMPLE_THREADS = 256;

__global__ __launch_bounds__(EDGE_SAMPLE_THREADS) void k_edge_sample(
    const float *__restrict__ x, int64_t rs, int64_t cs, int64_t step, uint32_t ns, uint32_t cap,
    const uint8_t *__restrict__ is_cat, uint32_t *__restrict__ keys) {
    const int f = blockIdx.y;
    const uint32_t s = blockIdx.x * EDGE_SAMPLE_THREADS + threadIdx.x;
    if (is_cat[f] || s >= ns) return;
    const float v = x[(int64_t)s * step * rs + (int64_t)f * cs];
    keys[(size_t)f * cap + s] = isnan(v) ? 0xFFFFFFFFu : float_key(v);
}

// Stable LSD radix sort of each column's n sample keys, 4-bit digits, 8
// passes, a column's keys split into B position chunks, one 1024-thread
// workgroup per (chunk, column).  Each pass is two launches: k_edge_count
// counts every chunk's digits, then k_edge_pass scatters.  A chunk's keys go
// in tiles of 8,192 (8 per thread: key tile + j * 1024 + thread), the next
// tile's keys loading while one is ranked; a key's rank among equal digits in
// its wavefront comes from four ballots, and tiles, j, wavefronts and lanes
// keep the input order.  A digit's keys from chunk c start after every
// smaller digit's keys and after the same digit's keys of chunks < c, so each
// pass is stable.  Behind each column's n keys, keys_a holds the chunk counts
// of the current pass and keys_b the NaN counts of the first.
constexpr int ESORT_KPT = 8;
constexpr uint32_t ESORT_TILE = EDGE_THREADS * ESORT_KPT;
constexpr uint32_t ESORT_MAX_CHUNKS = 32;
constexpr uint32_t ESORT_SCRATCH = 16 * ESORT_MAX_CHUNKS;   // words behind a column's keys

// Per-wavefront digit match of lane's digit d among the valid lanes.
__device__ __forceinline__ uint64_t digit_match(uint32_t d, uint64_t valid) {
    uint64_t m = valid;
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
        const uint64_t bb = __ballot((d >> bt) & 1u);
        m &= ((d >> bt) & 1u) ? bb : ~bb;
    }
    return m;
}

// The 8 keys of tile t0 for this thread (0 at or past end).
__device__ __forceinline__ void esort_load(const uint32_t *src, uint32_t t0, uint32_t end, int tid,
                                           uint32_t (&k)[ESORT_KPT]) {
#pragma unroll
    for (int j = 0; j < ESORT_KPT; ++j) {
        const uint32_t i = t0 + (uint32_t)j * EDGE_THREADS + (uint32_t)tid;
        k[j] = i < end ? src[i] : 0u;
    }
}

// Digit `pass` counts of chunk blockIdx.x of column blockIdx.y (and, on the
// first pass, its NaN keys), read from the pass's input (keys_a for even
// passes).
__global__ __launch_bounds__(EDGE_THREADS) void k_edge_count(uint32_t *__restrict__ keys_a,
                                                             uint32_t *__restrict__ keys_b,
                                                             uint32_t cap, uint32_t n,
                                                             uint32_t chunk, int pass,
                                                             const uint8_t *__restrict__ is_cat) {
    __shared__ uint32_t hist[16], s_nan;
    const int f = blockIdx.y, tid = threadIdx.x, lane = lane_id();
    if (is_cat[f]) return;
    const int shift = pass * 4;
    const uint32_t c = blockIdx.x, c0 = c * chunk, c1 = min(n, c0 + chunk);
    if (tid < 16) hist[tid] = 0;
    if (tid == 0) s_nan = 0;
    __syncthreads();
    const uint32_t *src = ((pass & 1) == 0 ? keys_a : keys_b) + (size_t)f * cap;
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    uint32_t nanc = 0, cur[ESORT_KPT], nxt[ESORT_KPT];
    esort_load(src, c0, c1, tid, nxt);
    for (uint32_t t0 = c0; t0 < c1; t0 += ESORT_TILE) {
#pragma unroll
        for (int j = 0; j < ESORT_KPT; ++j) cur[j] = nxt[j];
        if (t0 + ESORT_TILE < c1) esort_load(src, t0 + ESORT_TILE, c1, tid, nxt);
#pragma unroll
        for (int j = 0; j < ESORT_KPT; ++j) {
            const bool valid = t0 + (uint32_t)j * EDGE_THREADS + (uint32_t)tid < c1;
            if (pass == 0 && valid && cur[j] == 0xFFFFFFFFu) ++nanc;
            const uint32_t d = (cur[j] >> shift) & 15u;
            const uint64_t m = digit_match(d, __ballot(valid));
            if (valid && (m & lt) == 0) atomicAdd(&hist[d], (uint32_t)__popcll(m));
        }
    }
    if (pass == 0) {
        nanc = wave_sum(nanc);
        if (lane == 0 && nanc) atomicAdd(&s_nan, nanc);
    }
    __syncthreads();
    uint32_t *cnt = keys_a + (size_t)f * cap + n;
    if (tid < 16) cnt[c * 16 + tid] = hist[tid];
    if (pass == 0 && tid == 0) keys_b[(size_t)f * cap + n + c] = s_nan;
}

// One pass: scatter chunk blockIdx.x of column blockIdx.y by digit `pass`
// from the pass's input (keys_a for even passes) to the other buffer.
__global__ __launch_bounds__(EDGE_THREADS) void k_edge_pass(uint32_t *__restrict__ keys_a,
                                                            uint32_t *__restrict__ keys_b,
                                                            uint32_t cap, uint32_t n,
                                                            uint32_t chunk, uint32_t nchunks,
                                                            int pass,
                                                            const uint8_t *__restrict__ is_cat) {
    __shared__ uint32_t hist[16];
    __shared__ uint32_t cc[ESORT_MAX_CHUNKS][16];
    __shared__ uint32_t cnt[ESORT_KPT][EDGE_WAVES][16];   // leaders' counts, then offsets
    __shared__ uint32_t tot[ESORT_KPT][16];
    const int f = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = lane_id();
    if (is_cat[f]) return;
    const int shift = pass * 4;
    const bool even = (pass & 1) == 0;
    const uint32_t *src = (even ? keys_a : keys_b) + (size_t)f * cap;
    uint32_t *dst = (even ? keys_b : keys_a) + (size_t)f * cap;
    const uint32_t c = blockIdx.x, c0 = c * chunk, c1 = min(n, c0 + chunk);
    // this chunk's first slot per digit, from every chunk's counts
    const uint32_t *counts = keys_a + (size_t)f * cap + n;
    for (uint32_t k = tid; k < nchunks * 16; k += EDGE_THREADS) (&cc[0][0])[k] = counts[k];
    __syncthreads();
    if (tid < 16) {
        uint32_t total = 0, before = 0;
        for (uint32_t q = 0; q < nchunks; ++q) {
            total += cc[q][tid];
            if (q < c) before += cc[q][tid];
        }
        tot[0][tid] = total;
        hist[tid] = before;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        for (int d = 0; d < 16; ++d) {
            hist[d] += acc;
            acc += tot[0][d];
        }
    }
    __syncthreads();
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    uint32_t key[ESORT_KPT], nxt[ESORT_KPT];
    esort_load(src, c0, c1, tid, nxt);
    for (uint32_t t0 = c0; t0 < c1; t0 += ESORT_TILE) {
        uint32_t rank[ESORT_KPT];
        bool valid[ESORT_KPT];
#pragma unroll
        for (int j = 0; j < ESORT_KPT; ++j) key[j] = nxt[j];
        if (t0 + ESORT_TILE < c1) esort_load(src, t0 + ESORT_TILE, c1, tid, nxt);
        for (int k = tid; k < ESORT_KPT * EDGE_WAVES * 16; k += EDGE_THREADS)
            (&cnt[0][0][0])[k] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ESORT_KPT; ++j) {
            valid[j] = t0 + (uint32_t)j * EDGE_THREADS + (uint32_t)tid < c1;
            const uint32_t d = (key[j] >> shift) & 15u;
            const uint64_t m = digit_match(d, __ballot(valid[j]));
            rank[j] = (uint32_t)__popcll(m & lt);
            if (valid[j] && rank[j] == 0) cnt[j][w][d] = (uint32_t)__popcll(m);
        }
        __syncthreads();
        // offsets: within each (j, d), wavefronts in order ...
        if (tid < ESORT_KPT * 16) {
            const int j = tid >> 4, d = tid & 15;
            uint32_t acc = 0;
            for (int ww = 0; ww < EDGE_WAVES; ++ww) {
                const uint32_t v = cnt[j][ww][d];
                cnt[j][ww][d] = acc;
                acc += v;
            }
            tot[j][d] = acc;
        }
        __syncthreads();
        // ... then j in order, from the digit's next free slot
        if (tid < 16) {
            uint32_t acc = hist[tid];
            for (int j = 0; j < ESORT_KPT; ++j) {
                const uint32_t v = tot[j][tid];
                tot[j][tid] = acc;
                acc += v;
            }
            hist[tid] = acc;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ESORT_KPT; ++j) {
            if (!valid[j]) continue;
            const uint32_t d = (key[j] >> shift) & 15u;
            const uint32_t pos = tot[j][d] + cnt[j][w][d] + rank[j];
            if (pos < n) dst[pos] = key[j];          // always, with consistent counts
        }
        __syncthreads();                             // cnt / tot reuse by the next tile
    }
}

// Edge k = sorted[min(m - 1, (k + 1) * m / dataBins)] of the m non-NaN
// sample keys (0 for categorical or all-NaN columns); after the 8 passes the
// sorted keys are in keys_a.
__global__ void k_edge_pick(const uint32_t *__restrict__ keys_a,
                            const uint32_t *__restrict__ keys_b, uint32_t cap, uint32_t n,
                            uint32_t nchunks, const uint8_t *is_cat, int32_t num_bins,
                            float *__restrict__ edges) {
    __shared__ uint32_t s_m;
    const int f = blockIdx.x;
    const int data_bins = num_bins - 1, ne = data_bins - 1;
    if (threadIdx.x == 0) {
        uint32_t nan = 0;
        if (!is_cat[f])
            for (uint32_t c = 0; c < nchunks; ++c)
                nan += keys_b[(size_t)f * cap + n + c];
        s_m = is_cat[f] ? 0u : n - nan;
    }
    __syncthreads();
    const int64_t m = s_m;
    const uint32_t *keys = keys_a + (size_t)f * cap;
    for (int k = threadIdx.x; k < ne; k += blockDim.x) {
        float e = 0.0f;
        if (m > 0) {
            int64_t idx = ((int64_t)(k + 1) * m) / data_bins;
            if (idx > m - 1) idx = m - 1;
            e = key_float(keys[idx]);
        }
        edges[(size_t)f * ne + k] = e;
    }
}

// Samples of a column: rows 0, step, 2 step, ... with step = rows / 200000.
static int64_t edge_step(int64_t rows) { return rows / 200000 < 1 ? 1 : rows / 200000; }

size_t edge_sample_cap(int64_t rows) {
    const int64_t step = edge_step(rows);
    return (size_t)((rows + step - 1) / step) + ESORT_SCRATCH;
}

hipError_t launch_edges(hipStream_t s, const float *x, int64_t rows, int32_t cols, int64_t rs,
                        int64_t cs, int32_t num_bins, const uint8_t *is_cat, uint32_t *keys_a,
                        uint32_t *keys_b, uint32_t *counts, float *edges) {
    (void)counts;
    if (rows <= 0 || cols <= 0 || cols > 65535) return hipErrorInvalidValue;
    const int64_t step = edge_step(rows);
    const uint32_t cap = (uint32_t)edge_sample_cap(rows);
    const uint32_t ns = (uint32_t)((rows + step - 1) / step);
    // chunks per column: about 512 workgroups per pass (2048 measured slower:
    // per-workgroup set-up), each at least one tile
    uint32_t nch = (uint32_t)std::max(1, 512 / cols);
    nch = std::min(nch, std::min(ESORT_MAX_CHUNKS, (ns + ESORT_TILE - 1) / ESORT_TILE));
    const uint32_t chunk = (ns + nch - 1) / nch;
    nch = (ns + chunk - 1) / chunk;
    const dim3 sgrid((ns + EDGE_SAMPLE_THREADS - 1) / EDGE_SAMPLE_THREADS, (unsigned)cols);
    hipLaunchKernelGGL(k_edge_sample, sgrid, dim3(EDGE_SAMPLE_THREADS), 0, s, x, rs, cs, step, ns,
                       cap, is_cat, keys_a);
    const dim3 cgrid(nch, (unsigned)cols);
    for (int pass = 0; pass < 8; ++pass) {
        hipLaunchKernelGGL(k_edge_count, cgrid, dim3(EDGE_THREADS), 0, s, keys_a, keys_b, cap, ns,
                           chunk, pass, is_cat);
        hipLaunchKernelGGL(k_edge_pass, cgrid, dim3(EDGE_THREADS), 0, s, keys_a, keys_b, cap, ns,
                           chunk, nch, pass, is_cat);
    }
    hipLaunchKernelGGL(k_edge_pick, dim3(cols), dim3(256), 0, s, keys_a, keys_b, cap, ns, nch,
                       is_cat, num_bins, edges);
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

// Label (and weight) checks and the base score's sums over the training rows
// (validateLabels, Booster.swift:1724-1765; the mean of baseScore, :798-830).
// One wavefront per block of LABEL_BLOCK rows: lane l adds rows l, l + 64,
// ... of the block in order in double, then the 64 lane sums meet in a fixed
// tree (lane l adds lane l + s for s = 32, 16, ..., 1), so the block's sums
// do not depend on the schedule.  Per block: the two sums (logistic: the
// positive and total weight, scale_pos_weight applied; otherwise the weighted
// label sum and total weight) and the first row whose label, or weight, the
// objective rejects.
constexpr int64_t LABEL_BLOCK = 65536;

constexpr int LABEL_BATCH = 16;                      // rows per lane in flight

__global__ __launch_bounds__(64) void k_label_stats(int32_t obj, int32_t num_classes,
                                                    const float *__restrict__ y,
                                                    const float *__restrict__ w, int64_t n,
                                                    float spw, LabelStats *__restrict__ out) {
    constexpr int32_t LOGISTIC = 1, POISSON = 5, TWEEDIE = 6, MULTICLASS = 7;
    constexpr int64_t STEPS = LABEL_BLOCK / 64;
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * LABEL_BLOCK;
    const double sp = (double)spw;
    double a1 = 0.0, a2 = 0.0;
    int64_t bad_y = INT64_MAX, bad_w = INT64_MAX;
    // the lane's rows r0 + k * 64 + lane, k = 0, 1, ... in batches, the next
    // batch loading while one is added (in row order)
    float yn[LABEL_BATCH], wn[LABEL_BATCH];
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int j = 0; j < LABEL_BATCH; ++j) {
            const int64_t i = r0 + (k0 + j) * 64 + lane;
            yn[j] = i < n ? y[i] : 0.0f;
            wn[j] = (w && i < n) ? w[i] : 1.0f;
        }
    };
    load(0);
    for (int64_t k0 = 0; k0 < STEPS && r0 + k0 * 64 < n; k0 += LABEL_BATCH) {
        float yc[LABEL_BATCH], wc[LABEL_BATCH];
#pragma unroll
        for (int j = 0; j < LABEL_BATCH; ++j) { yc[j] = yn[j]; wc[j] = wn[j]; }
        if (k0 + LABEL_BATCH < STEPS) load(k0 + LABEL_BATCH);
#pragma unroll
        for (int j = 0; j < LABEL_BATCH; ++j) {
            const int64_t i = r0 + (k0 + j) * 64 + lane;
            if (i >= n) break;
            const float v = yc[j];
            bool ok = isfinite(v);
            if (obj == LOGISTIC) ok = ok && (v == 0.0f || v == 1.0f);
            if (obj == POISSON || obj == TWEEDIE) ok = ok && v >= 0.0f;
            if (obj == MULTICLASS) {
                const float r = rintf(v);
                ok = ok && r == v && r >= 0.0f && (int64_t)r < num_classes;
            }
            if (!ok && bad_y == INT64_MAX) bad_y = i;
            double wd = 1.0;
            if (w) {
                const float wf = wc[j];
                if (!(isfinite(wf) && wf >= 0.0f) && bad_w == INT64_MAX) bad_w = i;
                wd = (double)wf;
            }
            if (obj == LOGISTIC) {
                if (v > 0.5f) {
                    a1 += wd * sp;
                    a2 += wd * sp;
                } else {
                    a2 += wd;
                }
            } else {
                a1 += wd * (double)v;
                a2 += wd;
            }
        }
    }
    for (int s = 32; s >= 1; s >>= 1) {
        a1 += __shfl_down(a1, s, 64);
        a2 += __shfl_down(a2, s, 64);
        bad_y = min(bad_y, (int64_t)__shfl_down(bad_y, s, 64));
        bad_w = min(bad_w, (int64_t)__shfl_down(bad_w, s, 64));
    }
    if (lane == 0) out[blockIdx.x] = LabelStats{a1, a2, bad_y, bad_w};
}

size_t label_stats_blocks(int64_t rows) { return (size_t)((rows + LABEL_BLOCK - 1) / LABEL_BLOCK); }

hipError_t launch_label_stats(hipStream_t s, int32_t objective, int32_t num_classes,
                              const float *y, const float *w, int64_t rows, float spw,
                              LabelStats *out) {
    if (rows <= 0) return hipSuccess;
    const size_t blocks = label_stats_blocks(rows);
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_label_stats, dim3((unsigned)blocks), dim3(64), 0, s, objective,
                       num_classes, y, w, rows, spw, out);
    return hipGetLastError();
}

// max |g| and max h as f32 bit patterns (reduce_max_gh, Shaders.swift:87-94).
// Stage 1 (k_grad_max): grad_max_blocks(rows) blocks of 256 threads, one
// 16-B quad of rows per thread and step, one partial pair per block; with
// STORE every row's g and h also go to g_out / h_out (a sampled tree's later
// passes read them).  Stage 2 (k_grad_max_final): one wavefront reduces the
// partial pairs into the control block.  (Folding stage 2 into the next
// kernel's blocks was measured slower: each block then waits for the
// partials before its first load.)
constexpr int GRAD_THREADS = 256;
constexpr int GRAD_MAX_BLOCKS = 1024;
constexpr int SAMPLE_MAX_BLOCKS = 4096;   // partial maxima of the row-sampling pass

__device__ __forceinline__ void grad_max_row(const GradParams &gp, float p, float y, float w,
                                             uint32_t &mg, uint32_t &mh, float &g, float &h) {
    row_grad(gp, p, y, w, g, h);
    mg = max(mg, __float_as_uint(fabsf(g)));
    mh = max(mh, __float_as_uint(h));
}

// (max over n pairs of partial[2k], max of partial[2k+1]) for every thread of
// the block: wave 0 reduces, LDS broadcasts.
__device__ __forceinline__ uint2 reduce_partial_max(const uint32_t *__restrict__ partial, int n,
                                                    uint2 *s_bcast) {
    if (threadIdx.x < 64) {
        uint32_t a = 0, b = 0;
        for (int k = (int)threadIdx.x; k < n; k += 64) {
            a = max(a, partial[2 * k]);
            b = max(b, partial[2 * k + 1]);
        }
        a = wave_max_u32(a);
        b = wave_max_u32(b);
        if (threadIdx.x == 0) *s_bcast = make_uint2(a, b);
    }
    __syncthreads();
    return *s_bcast;
}

template <bool VEC, bool STORE>   // VEC: 16B-aligned inputs, four rows per load
__global__ __launch_bounds__(GRAD_THREADS) void k_grad_max(GradParams gp,
                                                           const float *__restrict__ preds,
                                                           const float *__restrict__ labels,
                                                           const float *__restrict__ weights,
                                                           int64_t rows,
                                                           uint32_t *__restrict__ partial,
                                                           float *__restrict__ g_out,
                                                           float *__restrict__ h_out) {
    __shared__ uint32_t red[2][GRAD_THREADS / 64];
    uint32_t mg = 0, mh = 0;
    const int64_t n4 = VEC ? rows >> 2 : 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const float4 *p4 = reinterpret_cast<const float4 *>(preds);
    const float4 *y4 = reinterpret_cast<const float4 *>(labels);
    const float4 *w4 = reinterpret_cast<const float4 *>(weights);
    const float4 one = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    auto quad = [&](int64_t q, const float4 &p, const float4 &y, const float4 &w) {
        float4 g, h;
        grad_max_row(gp, p.x, y.x, w.x, mg, mh, g.x, h.x);
        grad_max_row(gp, p.y, y.y, w.y, mg, mh, g.y, h.y);
        grad_max_row(gp, p.z, y.z, w.z, mg, mh, g.z, h.z);
        grad_max_row(gp, p.w, y.w, w.w, mg, mh, g.w, h.w);
        if (STORE) {
            reinterpret_cast<float4 *>(g_out)[q] = g;
            reinterpret_cast<float4 *>(h_out)[q] = h;
        }
    };
    for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < n4; q += stride)
        quad(q, p4[q], y4[q], gp.has_weights ? w4[q] : one);
    // rows not covered by the 16B loads (all of them when !VEC)
    for (int64_t i = (n4 << 2) + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < rows;
         i += stride) {
        float g, h;
        row_grad_at(gp, preds, labels, weights, i, g, h);
        mg = max(mg, __float_as_uint(fabsf(g)));
        mh = max(mh, __float_as_uint(h));
        if (STORE) { g_out[i] = g; h_out[i] = h; }
    }
    mg = wave_max_u32(mg);
    mh = wave_max_u32(mh);
    const int w = threadIdx.x >> 6;
    if (lane_id() == 0) { red[0][w] = mg; red[1][w] = mh; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t a = red[0][0], b = red[1][0];
        for (int k = 1; k < GRAD_THREADS / 64; ++k) { a = max(a, red[0][k]); b = max(b, red[1][k]); }
        partial[2 * blockIdx.x] = a;
        partial[2 * blockIdx.x + 1] = b;
    }
}

__global__ __launch_bounds__(64) void k_grad_max_final(const uint32_t *__restrict__ partial,
                                                       int nblocks, TreeCtl *ctl) {
    __shared__ uint2 bc;
    const uint2 m = reduce_partial_max(partial, nblocks, &bc);
    if (threadIdx.x == 0) {
        ctl->max_gh[0] = m.x;
        ctl->max_gh[1] = m.y;
    }
}

// A tree's start in one single-wavefront launch: the previous tree's control
// block copied to ctl_out (when given), the block zeroed, and (with partial)
// the gradient maxima reduced into it as k_grad_max_final does.
static_assert(sizeof(TreeCtl) % 4 == 0 && sizeof(TreeCtl) / 4 <= 64, "one word per lane");

__global__ __launch_bounds__(64) void k_tree_start(TreeCtl *ctl, TreeCtl *ctl_out,
                                                   const uint32_t *__restrict__ partial,
                                                   int nparts) {
    constexpr uint32_t CW = sizeof(TreeCtl) / 4;
    uint32_t *w = reinterpret_cast<uint32_t *>(ctl);
    if (threadIdx.x < CW) {
        const uint32_t v = w[threadIdx.x];           // each lane owns one word
        if (ctl_out) reinterpret_cast<uint32_t *>(ctl_out)[threadIdx.x] = v;
        w[threadIdx.x] = 0u;
    }
    if (partial) {
        __shared__ uint2 bc;
        const uint2 m = reduce_partial_max(partial, nparts, &bc);
        if (threadIdx.x == 0) {                      // after lanes 0 and 1 zeroed these words
            ctl->max_gh[0] = m.x;
            ctl->max_gh[1] = m.y;
        }
    }
}

hipError_t launch_tree_start(hipStream_t s, TreeCtl *ctl, TreeCtl *ctl_out,
                             const uint32_t *partial, int nparts) {
    hipLaunchKernelGGL(k_tree_start, dim3(1), dim3(64), 0, s, ctl, ctl_out, partial,
                       partial ? nparts : 0);
    return hipGetLastError();
}

static int grad_max_blocks(int64_t rows) {
    const int64_t quads = (rows + 3) / 4;
    return (int)std::max<int64_t>(
        1, std::min<int64_t>(GRAD_MAX_BLOCKS, (quads + GRAD_THREADS - 1) / GRAD_THREADS));
}

hipError_t launch_grad_max(hipStream_t s, const GradParams &gp, const float *preds,
                           const float *labels, const float *weights, int64_t rows,
                           TreeCtl *ctl, uint32_t *partial, float *g_out, float *h_out) {
    const int blocks = grad_max_blocks(rows);
    const bool store = g_out != nullptr && h_out != nullptr;
    const bool vec = gp.objective != 7 &&
                     ((reinterpret_cast<uintptr_t>(preds) | reinterpret_cast<uintptr_t>(labels) |
                       reinterpret_cast<uintptr_t>(weights) | reinterpret_cast<uintptr_t>(g_out) |
                       reinterpret_cast<uintptr_t>(h_out)) & 15u) == 0;
    auto kernel = vec ? (store ? k_grad_max<true, true> : k_grad_max<true, false>)
                      : (store ? k_grad_max<false, true> : k_grad_max<false, false>);
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(GRAD_THREADS), 0, s, gp, preds, labels,
                       weights, rows, partial, g_out, h_out);
    hipLaunchKernelGGL(k_grad_max_final, dim3(1), dim3(64), 0, s, partial, blocks, ctl);
    return hipGetLastError();
}

hipError_t launch_grad_max_final(hipStream_t s, const uint32_t *partial, int nparts,
                                 TreeCtl *ctl) {
    hipLaunchKernelGGL(k_grad_max_final, dim3(1), dim3(64), 0, s, partial, nparts, ctl);
    return hipGetLastError();
}

size_t grad_max_scratch_words() { return 2 * (size_t)std::max(GRAD_MAX_BLOCKS, SAMPLE_MAX_BLOCKS); }

// ---------------------------------------------------------------------------
// row sampling: GOSS and bagging (goss_grad_hist, goss_threshold, goss_select,
// Shaders.swift:1093-1199, driven as in Booster.swift:1401-1445).
// The tree's gradients come from the maxima pass (launch_grad_max with
// g_out / h_out), so the passes below stream 4-8 B per row and compute no
// gradient: with the logistic objective's double-precision exp, recomputing
// g per pass cost more than reading it back.
// ---------------------------------------------------------------------------

constexpr int GOSS_BUCKETS = 1024;

__device__ __forceinline__ uint32_t wang_hash(uint32_t x) {
    x = (x ^ 61u) ^ (x >> 16);
    x *= 9u;
    x ^= x >> 4;
    x *= 0x27d4eb2du;
    x ^= x >> 15;
    return x;
}

// |g| / max|g| histogram in 1024 buckets: one LDS sub-histogram per
// wavefront (|g| clusters early in training, and same-bucket adds from
// different wavefronts would serialize), merged with one global add per
// non-empty bucket and block.  Adds to one global address serialize (about
// 11 ns each on MI355X), so the grid is a few large blocks: GOSS_HIST_BLOCKS
// of 1024 threads, grid-stride over 16-B quads of g with two in flight per
// thread; the rows % 4 tail one per thread.
constexpr int GOSS_HIST_THREADS = 1024;
constexpr int GOSS_HIST_BLOCKS = 256;

__global__ __launch_bounds__(GOSS_HIST_THREADS) void k_goss_hist(const float *__restrict__ g,
                                                                 int64_t rows, TreeCtl *ctl,
                                                                 uint32_t *buckets,
                                                                 TreeCtl *ctl_out,
                                                                 const uint32_t *walk_part,
                                                                 int walk_nparts) {
    constexpr int WAVES = GOSS_HIST_THREADS / 64;
    __shared__ uint32_t lb[WAVES][GOSS_BUCKETS];
    for (int k = threadIdx.x; k < WAVES * GOSS_BUCKETS; k += blockDim.x) (&lb[0][0])[k] = 0;
    if (walk_part && blockIdx.x == 0 && threadIdx.x < sizeof(TreeCtl) / 4) {
        // the tree's start (k_tree_start): the previous tree's control block
        // copied out, this one zeroed; its maxima are stored below
        uint32_t *w = reinterpret_cast<uint32_t *>(ctl);
        const uint32_t v = w[threadIdx.x];
        if (ctl_out) reinterpret_cast<uint32_t *>(ctl_out)[threadIdx.x] = v;
        w[threadIdx.x] = 0u;
    }
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const float4 *g4 = reinterpret_cast<const float4 *>(g);
    const int64_t nq = rows >> 2;
    // the first two quads load while the maxima are found
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const bool first = t0 < nq, second = t0 + stride < nq;
    const float4 a0 = first ? g4[t0] : zero4;
    const float4 b0 = second ? g4[t0 + stride] : zero4;
    float mg;
    if (walk_part) {
        // max |g| from the training walk's per-block maxima, in every block
        __shared__ uint2 bc;
        const uint2 m = reduce_partial_max(walk_part, walk_nparts, &bc);
        if (blockIdx.x == 0 && threadIdx.x == 0) {   // after the zeroing (barrier above)
            ctl->max_gh[0] = m.x;
            ctl->max_gh[1] = m.y;
        }
        mg = f32_from_bits(m.x);
    } else {
        __syncthreads();
        mg = f32_from_bits(ctl->max_gh[0]);
    }
    uint32_t *mine = lb[threadIdx.x >> 6];
    auto add = [&](float v) {
        const uint32_t b = (uint32_t)(fabsf(v) / mg * (float)GOSS_BUCKETS);
        atomicAdd(&mine[min(b, (uint32_t)(GOSS_BUCKETS - 1))], 1u);
    };
    if (mg > 0.0f) {
        if (first) { add(a0.x); add(a0.y); add(a0.z); add(a0.w); }
        if (second) { add(b0.x); add(b0.y); add(b0.z); add(b0.w); }
        for (int64_t q = t0 + 2 * stride; q < nq; q += 2 * stride) {
            const bool sec = q + stride < nq;
            const float4 a = g4[q];
            float4 b = zero4;
            if (sec) b = g4[q + stride];
            add(a.x); add(a.y); add(a.z); add(a.w);
            if (sec) { add(b.x); add(b.y); add(b.z); add(b.w); }
        }
        for (int64_t i = (nq << 2) + t0; i < rows; i += stride) add(g[i]);
    }
    __syncthreads();
    for (int k = threadIdx.x; k < GOSS_BUCKETS; k += blockDim.x) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) c += lb[w][k];
        if (c) atomicAdd(&buckets[k], c);
    }
}

// Threshold = lower edge of the bucket where the count from the top first
// reaches top_count (b = 1024, i.e. max|g|, when top_count = 0); the value
// is f32 bits.  Run by one whole wavefront.
__device__ uint32_t goss_threshold(uint32_t top_count, float mg,
                                   const uint32_t *__restrict__ buckets) {
    const int lane = lane_id();
    constexpr int PER = GOSS_BUCKETS / 64;
    uint32_t v[PER], s = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) { v[j] = buckets[lane * PER + j]; s += v[j]; }
    // suffix sums over lanes: from this lane's first bucket to the top
    uint32_t suf = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_down(suf, o, 64);
        if (lane + o < 64) suf += t;
    }
    uint32_t b = GOSS_BUCKETS;
    if (top_count > 0 && mg > 0.0f) {
        // the crossing lane: the highest lane whose suffix reaches top_count
        const uint64_t ok = __ballot(suf >= top_count);
        if (ok == 0) {
            b = 0;                                   // the whole histogram is below top_count
        } else {
            const int L = 63 - __builtin_clzll(ok);
            const uint32_t above = __shfl(suf - s, L, 64);   // count in lanes above L
            uint32_t cum = above, bb = (uint32_t)(L * PER + PER);
            uint32_t w[PER];
#pragma unroll
            for (int j = 0; j < PER; ++j) w[j] = __shfl(v[j], L, 64);
#pragma unroll
            for (int j = PER - 1; j >= 0; --j) {
                if (cum < top_count) { bb -= 1; cum += w[j]; }
            }
            b = bb;
        }
    }
    const float thr = mg > 0.0f ? (float)b / (float)GOSS_BUCKETS * mg : 0.0f;
    return __float_as_uint(thr);
}

// Entries move as one 64-bit word (row low, ghq high).  Order buffers are
// written once per pass and read by the next kernels from HBM (80 MB at 10M
// rows, far past L2), so their stores and the partition's loads are
// nontemporal: they do not displace the lines the histogram kernel's two tile
// workgroups share (measured: 3-4% per tree).
__device__ __forceinline__ void store_entry_nt(Entry *p, const Entry e) {
    __builtin_nontemporal_store((unsigned long long)e.row | ((unsigned long long)e.ghq << 32),
                                reinterpret_cast<unsigned long long *>(p));
}

__device__ __forceinline__ Entry load_entry_nt(const Entry *p) {
    const unsigned long long v =
        __builtin_nontemporal_load(reinterpret_cast<const unsigned long long *>(p));
    return Entry{(uint32_t)v, (uint32_t)(v >> 32)};
}

// Keep rows with |g| >= threshold (weight 1) and a hashed uniform sample of
// the rest (weight sp.weight).  512 threads take a 16384-row chunk, thread t
// the quads k * 512 + t (k < 8) of g and h, so each load instruction reads
// 8 KiB of contiguous rows.  A thread keeps its 32 keep / amplified decisions
// as bit masks; the block scans the per-thread counts, takes one cursor add
// per chunk (adds to one address serialize, so chunks are large; 32768-row
// chunks of 1024 threads measured 0.7 ms per HIGGS-like GOSS fit slower),
// stages the kept rows' chunk offsets (14 bits, amplified flag in bit 15) in
// LDS and then writes, contiguously, the entries
// {row, f32 bits of g * w} and h_kept = h * w.  Each block's maxima of |g| * w
// and h * w go into ctl->sample_max (atomic max of f32 bits: the values are
// >= 0); with kept non-null, kept[i] = 1 for a kept row and 0 otherwise.
// The entry order inside a chunk follows the staging, not the row order;
// every consumer sums integers or partitions stably, so the tree does not
// depend on it.
constexpr int SEL_THREADS = 512;
constexpr int SEL_QUADS = 8;
constexpr int SEL_CHUNK = SEL_THREADS * SEL_QUADS * 4;
static_assert(SEL_CHUNK <= (1 << 15), "chunk offsets fit 15 bits");

__global__ __launch_bounds__(SEL_THREADS) void k_goss_select(
    SampleParams sp, const float *__restrict__ g, const float *__restrict__ h, int64_t rows,
    const uint32_t *__restrict__ buckets, TreeCtl *ctl, Entry *__restrict__ order,
    float *__restrict__ h_kept, uint8_t *__restrict__ kept) {
    __shared__ uint16_t s_off[SEL_CHUNK];
    __shared__ uint32_t s_wave[SEL_THREADS / 64];
    __shared__ uint32_t s_base, s_total, s_thr;
    __shared__ uint32_t red[2][SEL_THREADS / 64];
    const int tid = threadIdx.x, w = tid >> 6;
    // the keep threshold, from the unweighted max |g| and the |g| histogram
    // (every block derives it: no separate one-wavefront kernel)
    if (tid < 64) {
        const uint32_t t = goss_threshold(sp.goss ? sp.top_count : 0u,
                                          f32_from_bits(ctl->max_gh[0]), buckets);
        if (tid == 0) {
            s_thr = t;
            if (blockIdx.x == 0) ctl->sample_thr = t;
        }
    }
    __syncthreads();
    const float thr = f32_from_bits(s_thr);
    const uint32_t seed_mix = sp.seed * 0x9E3779B9u;
    const float4 *g4 = reinterpret_cast<const float4 *>(g);
    const float4 *h4 = reinterpret_cast<const float4 *>(h);
    uint32_t mg = 0, mh = 0;
    for (int64_t c0 = (int64_t)blockIdx.x * SEL_CHUNK; c0 < rows;
         c0 += (int64_t)gridDim.x * SEL_CHUNK) {
        uint32_t keep = 0, amp = 0;
#pragma unroll
        for (int k = 0; k < SEL_QUADS; ++k) {
            const int64_t r0 = c0 + (int64_t)(k * SEL_THREADS + tid) * 4;
            float gv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, hv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (r0 + 3 < rows) {
                const float4 a = g4[r0 >> 2], b = h4[r0 >> 2];
                gv[0] = a.x; gv[1] = a.y; gv[2] = a.z; gv[3] = a.w;
                hv[0] = b.x; hv[1] = b.y; hv[2] = b.z; hv[3] = b.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (r0 + j < rows) { gv[j] = g[r0 + j]; hv[j] = h[r0 + j]; }
            }
            uint32_t nib = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t i = r0 + j;
                if (i >= rows) continue;
                const float ag = fabsf(gv[j]);
                float wt = 1.0f;
                bool kp = ag >= thr;
                if (!kp) {
                    const uint32_t hs = wang_hash((uint32_t)i ^ seed_mix);
                    if ((float)(hs >> 8) * (1.0f / 16777216.0f) < sp.other_prob) {
                        kp = true;
                        wt = sp.weight;
                    }
                }
                if (kp) {
                    nib |= 1u << j;
                    if (wt != 1.0f) amp |= 1u << (4 * k + j);
                    mg = max(mg, __float_as_uint(ag * wt));
                    mh = max(mh, __float_as_uint(hv[j] * wt));
                }
            }
            keep |= nib << (4 * k);
            if (kept) {
                if (r0 + 3 < rows) {
                    *reinterpret_cast<uint32_t *>(kept + r0) =
                        (nib & 1u) | ((nib >> 1) & 1u) << 8 | ((nib >> 2) & 1u) << 16 |
                        ((nib >> 3) & 1u) << 24;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (r0 + j < rows) kept[r0 + j] = (uint8_t)((nib >> j) & 1u);
                }
            }
        }
        // block-exclusive position of this thread's first kept row
        const uint32_t cnt = (uint32_t)__popc(keep);
        const uint32_t inc = wave_inclusive_scan(cnt);
        if (lane_id() == 63) s_wave[w] = inc;
        __syncthreads();
        if (tid == 0) {
            uint32_t acc = 0;
#pragma unroll
            for (int v = 0; v < SEL_THREADS / 64; ++v) {
                const uint32_t t = s_wave[v];
                s_wave[v] = acc;
                acc += t;
            }
            s_total = acc;
            s_base = atomicAdd(&ctl->sampled, acc);
        }
        __syncthreads();
        uint32_t pos = s_wave[w] + inc - cnt;
        for (uint32_t m = keep; m; m &= m - 1) {
            const uint32_t b = (uint32_t)__builtin_ctz(m);
            const uint32_t off = ((b >> 2) * SEL_THREADS + (uint32_t)tid) * 4u + (b & 3u);
            s_off[pos++] = (uint16_t)(off | (((amp >> b) & 1u) << 15));
        }
        __syncthreads();
        const uint32_t total = s_total, base = s_base;
        for (uint32_t q = (uint32_t)tid; q < total; q += SEL_THREADS) {
            const uint32_t v = s_off[q];
            const int64_t i = c0 + (v & 0x7FFFu);
            float gw = g[i], hw = h[i];              // this chunk's lines: still in L2
            if (v >> 15) { gw = gw * sp.weight; hw = hw * sp.weight; }
            store_entry_nt(order + base + q, Entry{(uint32_t)i, __float_as_uint(gw)});
            __builtin_nontemporal_store(hw, h_kept + base + q);
        }
        __syncthreads();                             // s_off / s_wave reuse by the next chunk
    }
    mg = wave_max_u32(mg);
    mh = wave_max_u32(mh);
    if (lane_id() == 0) { red[0][w] = mg; red[1][w] = mh; }
    __syncthreads();
    if (tid == 0) {
        uint32_t a = red[0][0], b = red[1][0];
        for (int k = 1; k < SEL_THREADS / 64; ++k) { a = max(a, red[0][k]); b = max(b, red[1][k]); }
        if (a) atomicMax(&ctl->sample_max[0], a);
        if (b) atomicMax(&ctl->sample_max[1], b);
    }
}

__device__ void plan_root(const RootPlan &rp);

// Covers of the level's nodes from count; with zero_empty, empty nodes' leaves
// become 0 (final_fixup_node is k_final_fixup's per-node step).
__device__ __forceinline__ void final_fixup_node(const LevelArgs &la, const uint32_t *count,
                                                 const TreeOut &out, int zero_empty,
                                                 uint32_t local) {
    const uint32_t n = la.level_start + local;
    const uint32_t c = count[n];
    out.cover[n] = (float)c;
    if (c == 0 && zero_empty) out.leaf[n] = 0.0f;
}

// The root pass's first workgroup: the previous tree's fixup, then the root plan.
__device__ void root_pass_block0(const RootPlan &rp, int has_plan, const PendingFixup &fx) {
    if (fx.active)
        for (uint32_t k = threadIdx.x; k < fx.la.num_level; k += blockDim.x)
            final_fixup_node(fx.la, fx.count, fx.out, fx.zero_empty, k);
    if (has_plan) plan_root(rp);
}

// Quantise the kept entries with the weighted maxima (quantize_gradients,
// Shaders.swift:176-192, over amplified gradients): ghq holds g * w on entry.
// The selection left the maxima in ctl->sample_max; block 0 stores them as
// the tree's max_gh for the split search and zeroes the |g| histogram for
// the next tree.
__global__ __launch_bounds__(256) void k_quantize_sampled(TreeCtl *ctl,
                                                          uint32_t *__restrict__ buckets,
                                                          Entry *__restrict__ order,
                                                          const float *__restrict__ h_kept,
                                                          RootPlan rp, int has_plan,
                                                          PendingFixup fx) {
    if (blockIdx.x == 0) {
        for (int k = threadIdx.x; k < GOSS_BUCKETS; k += blockDim.x) buckets[k] = 0;
        root_pass_block0(rp, has_plan, fx);          // overlaps the other workgroups' rows
    }
    const uint32_t n = ctl->sampled;
    const uint32_t i0 = blockIdx.x * blockDim.x + threadIdx.x, step = gridDim.x * blockDim.x;
    Entry e0{0u, 0u};
    float hw0 = 0.0f;
    if (i0 < n) {
        e0 = load_entry_nt(order + i0);
        hw0 = __builtin_nontemporal_load(h_kept + i0);
    }
    const uint32_t mgb = ctl->sample_max[0], mhb = ctl->sample_max[1];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        ctl->max_gh[0] = mgb;
        ctl->max_gh[1] = mhb;
    }
    const float mg = f32_from_bits(mgb), mh = f32_from_bits(mhb);
    const float gscale = mg > 0.0f ? 32767.0f / mg : 0.0f;
    const float hscale = mh > 0.0f ? 127.0f / mh : 0.0f;
    for (uint32_t i = i0; i < n; i += step) {
        Entry e = e0;
        float hw = hw0;
        if (i != i0) {
            e = load_entry_nt(order + i);
            hw = __builtin_nontemporal_load(h_kept + i);
        }
        const float gw = __uint_as_float(e.ghq);
        const int qg = (int)rintf(gw * gscale);
        const uint32_t qh = (uint32_t)rintf(hw * hscale);
        e.ghq = ((uint32_t)(qg & 0xFFFF) << 16) | (qh & 0x7Fu);
        store_entry_nt(order + i, e);
    }
}

hipError_t launch_sample(hipStream_t s, const SampleParams &sp, int64_t rows, TreeCtl *ctl,
                         uint32_t *buckets, const float *g, const float *h,
                         Entry *order, float *h_kept, uint8_t *kept, const RootPlan *plan,
                         const PendingFixup *fix, TreeCtl *ctl_prev, const uint32_t *walk_part,
                         int walk_nparts) {
    if (((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(h)) & 15u) != 0)
        return hipErrorInvalidValue;                 // the passes read 16-B quads
    const int64_t quads = (rows + 3) / 4;
    const unsigned hist_blocks = (unsigned)std::max<int64_t>(
        1, std::min<int64_t>(GOSS_HIST_BLOCKS,
                             (quads + 2 * GOSS_HIST_THREADS - 1) / (2 * GOSS_HIST_THREADS)));
    if (sp.goss && sp.top_count > 0) {
        hipLaunchKernelGGL(k_goss_hist, dim3(hist_blocks), dim3(GOSS_HIST_THREADS), 0, s, g, rows,
                           ctl, buckets, ctl_prev, walk_part, walk_part ? walk_nparts : 0);
    } else if (walk_part) {
        hipLaunchKernelGGL(k_tree_start, dim3(1), dim3(64), 0, s, ctl, ctl_prev, walk_part,
                           walk_nparts);
    }
    const int64_t blocks = std::max<int64_t>(
        1, std::min<int64_t>((rows + SEL_CHUNK - 1) / SEL_CHUNK, SAMPLE_MAX_BLOCKS));
    hipLaunchKernelGGL(k_goss_select, dim3((unsigned)blocks), dim3(SEL_THREADS), 0, s, sp, g, h,
                       rows, buckets, ctl, order, h_kept, kept);
    // the kept count is known only on the device: a fixed grid strides over it
    // (a rows-sized grid of mostly idle blocks measured 7 us slower)
    const unsigned qblocks =
        (unsigned)std::max<int64_t>(1, std::min<int64_t>(2048, (rows + 255) / 256));
    hipLaunchKernelGGL(k_quantize_sampled, dim3(qblocks), dim3(256), 0, s, ctl, buckets, order,
                       h_kept, plan ? *plan : RootPlan{}, plan ? 1 : 0,
                       fix ? *fix : PendingFixup{});
    return hipGetLastError();
}

// Every row quantised (quantize_gradients, Shaders.swift:176-192) into the
// order entries {row, (qg & 0xFFFF) << 16 | qh}, one row per thread.
__global__ __launch_bounds__(256) void k_quantize(GradParams gp, const float *__restrict__ preds,
                                                  const float *__restrict__ labels,
                                                  const float *__restrict__ weights, int64_t rows,
                                                  const TreeCtl *ctl, Entry *__restrict__ order,
                                                  int implicit_rows, RootPlan rp, int has_plan,
                                                  PendingFixup fx) {
    if (blockIdx.x == 0) root_pass_block0(rp, has_plan, fx);   // overlaps the other workgroups
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    const float mg = f32_from_bits(ctl->max_gh[0]), mh = f32_from_bits(ctl->max_gh[1]);
    const float gscale = mg > 0.0f ? 32767.0f / mg : 0.0f;
    const float hscale = mh > 0.0f ? 127.0f / mh : 0.0f;
    float g, h;
    row_grad_at(gp, preds, labels, weights, i, g, h);
    const int qg = (int)rintf(g * gscale);
    const uint32_t qh = (uint32_t)rintf(h * hscale);
    const uint32_t ghq = ((uint32_t)(qg & 0xFFFF) << 16) | (qh & 0x7Fu);
    if (implicit_rows) {
        __builtin_nontemporal_store(ghq, reinterpret_cast<uint32_t *>(order) + i);
    } else {
        store_entry_nt(order + i, Entry{(uint32_t)i, ghq});
    }
}

hipError_t launch_quantize(hipStream_t s, const GradParams &gp, const float *preds,
                           const float *labels, const float *weights, int64_t rows,
                           const TreeCtl *ctl, Entry *order, bool implicit_rows,
                           const RootPlan *plan, const PendingFixup *fix) {
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, gp,
                       preds, labels, weights, rows, ctl, order, implicit_rows ? 1 : 0,
                       plan ? *plan : RootPlan{}, plan ? 1 : 0, fix ? *fix : PendingFixup{});
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// histograms: packed 64-bit LDS words, one item per (node chunk, tile)
//
// Every lane owns one row of the item and a plane of P = min(W, 32) features
// of that row (W = 64: two lanes per row, one per 32-feature half; W <= 32:
// one row per lane).  At step s (0 <= s < P) lane r adds its row's value to
// feature (r & (P-1)) ^ s of its plane, so the 32 lanes of each half-wave hit
// 32 distinct cells, one per bank pair, and the row's packed (qg, qh) word
// never leaves the lane.  (A ds_add_u64 is served one half-wave at a time:
// the two halves may share cells at no cost, while a 2-way bank conflict
// inside a half costs 30%.)  The LDS histogram is two planes of [256 bins][32
// columns] u64 (128 KiB); cell (plane, bin, column) sits at byte address
// plane*65536 + bin*256 + column*8, which one v_perm_b32 assembles from the
// bin byte and a per-lane column word.  Each lane gathers its P bytes with 16B
// loads whose chunk order, and then dword order, are permuted once per row so
// that step s reads a fixed register and byte.  Columns hold feature c (W = 64:
// 32*plane + c; W = 32: plane 0, shared by both halves) or copy c / W of
// feature c % W (W <= 16), summed when the item is flushed.
//
// Extras (W = 32, Shape::extras): tile t also adds E_t <= 2 features of the
// last layout tile, from one dword per row.  Plane 1 then holds 32 / E_t
// copies of them: at extra step j lane r adds to column (r & 31) ^ j, whose
// low bit (E_t = 2) names the extra feature, so each half-wave again hits 32
// distinct bank pairs.  Loads are pipelined: data three batches ahead,
// entries nine.
//
// Paired 32-wide tiles (W = 32, two lanes per row, for gathered rows): lane
// 2r + q holds features 16q .. 16q+15 of row r, so one 16-B load per lane
// brings the tile and a half-wave holds 16 rows x both halves.  At step s lane
// (r, q) adds feature 16q + ((r & 15) ^ s) to plane 0, column 16q + ((r & 15)
// ^ s): 32 distinct bank pairs per half-wave, 16 steps per 32 rows.  Extras
// (E_t <= 2) take one more step: lane (r, q) adds extra q to plane 1, column
// 16q + (r & 15), i.e. 16 copies per extra (lanes with q >= E_t fill columns
// of an extra the tile does not carry, which the flush never reads).
// ---------------------------------------------------------------------------

constexpr int HIST_THREADS = 1024;
constexpr int HIST_LDS_BYTES = 2 * 256 * 32 * 8;     // two planes of [256][32] u64, static
// ring depths chosen by measurement (3 / 9 beat 2..6 / 6..15 at 10M x 100:
// deeper data rings cost L2 reuse between the two tiles of a row)
// (per lanes-per-row mode below: 3 / 9 with two lanes per 64-wide row, 4 / 8
// with four; at four, 4 to 8 data batches measured the same)
template <int W, int LPR> constexpr int hist_data_ring() { return W / LPR == 16 ? 4 : 3; }
template <int W, int LPR> constexpr int hist_entry_ring() { return W / LPR == 16 ? 8 : 9; }
// true: the per-lane LDS column words sit in a 32-register table; false: each
// is rebuilt with one XOR per update (frees the table's registers)
constexpr bool HIST_COLW_TABLE = true;

// P bytes of one row as loaded: 16B chunks in the order (u ^ cx)
template <int P> struct RowRaw { uint32_t d[P / 4]; };

template <int P>
__device__ __forceinline__ RowRaw<P> load_row_raw(const uint8_t *src, uint32_t cx) {
    RowRaw<P> out;
    if constexpr (P == 8) {
        const uint2 v = *reinterpret_cast<const uint2 *>(src);
        out.d[0] = v.x;
        out.d[1] = v.y;
    } else {
#pragma unroll
        for (int u = 0; u < P / 16; ++u) {
            const uint4 v = *reinterpret_cast<const uint4 *>(src + 16u * ((uint32_t)u ^ cx));
            out.d[4 * u + 0] = v.x;
            out.d[4 * u + 1] = v.y;
            out.d[4 * u + 2] = v.z;
            out.d[4 * u + 3] = v.w;
        }
    }
    return out;
}

// dword order within each 16B chunk permuted by (m & 3): d'[v] = d[v ^ (m & 3)]
template <int P>
__device__ __forceinline__ RowRaw<P> permute_dwords(const RowRaw<P> &in, bool b0, bool b1) {
    RowRaw<P> out;
    if constexpr (P == 8) {
        out.d[0] = b0 ? in.d[1] : in.d[0];
        out.d[1] = b0 ? in.d[0] : in.d[1];
    } else {
#pragma unroll
        for (int u = 0; u < P / 16; ++u) {
            const uint32_t *v = in.d + 4 * u;
            const uint32_t x0 = b0 ? v[1] : v[0], x1 = b0 ? v[0] : v[1];
            const uint32_t x2 = b0 ? v[3] : v[2], x3 = b0 ? v[2] : v[3];
            out.d[4 * u + 0] = b1 ? x2 : x0;
            out.d[4 * u + 1] = b1 ? x3 : x1;
            out.d[4 * u + 2] = b1 ? x0 : x2;
            out.d[4 * u + 3] = b1 ? x1 : x3;
        }
    }
    return out;
}

// lay: where each tile's rows sit (the gather layout, or the planar root
// copy, whose last tile's loads run into the next row: those bytes land in
// padding columns, which are never reduced).
// IMPLICIT: order holds one u32 packed (qg, qh) per row of the root, entry j
// being row j (k_quantize's implicit form).
// LPR: lanes per row of a 64-wide tile.  2: 32 features per lane (the planar
// root, whose rows are contiguous); 4: 16 per lane, so one 16-B load
// instruction covers a gathered row's whole tile (-4% on deep levels at 10M x
// 100 against 2, which needs two).  32-wide tiles: 1 (one row per lane) or 2
// (paired, above).  Narrower tiles: one row per lane.
template <int W, int LPR, bool IMPLICIT>
__global__ __launch_bounds__(HIST_THREADS) void k_hist(const uint8_t *__restrict__ tiled,
                                                       const Entry *__restrict__ order,
                                                       const HistItem *__restrict__ items,
                                                       const TreeCtl *ctl,
                                                       uint64_t *__restrict__ partials,
                                                       HistLayout lay, Shape sh) {
    static_assert(W == 64   ? (LPR == 2 || LPR == 4)
                  : W == 32 ? (LPR == 1 || LPR == 2)
                            : LPR == 1,
                  "lanes per row");
    constexpr int P = W / LPR > 32 ? 32 : W / LPR;   // features per lane
    constexpr int RPB = 64 / LPR;                    // rows per wavefront batch
    constexpr bool XTRA = W == 32;                   // extras possible (plane 1 free)
    constexpr bool PAIRED = W == 32 && LPR == 2;     // lane 2r + q: row r, half q
    constexpr int DR = hist_data_ring<W, LPR>(), ER = hist_entry_ring<W, LPR>();
    static_assert(ER > DR, "a data refill needs the entry DR batches ahead");
    static_assert(ER % DR == 0, "batch k of every round uses data slot k % DR");
    constexpr int LDS_BYTES = HIST_LDS_BYTES;
    __shared__ uint64_t hist_lds[LDS_BYTES / 8];
    const int32_t nb = sh.num_bins, cols = sh.cols, PW = sh.part_w;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // scalar: loop bounds stay uniform
    const uint32_t nwaves = HIST_THREADS / 64;
    // lane = q * RPB + rl (paired: 2 * rl + q): row rl of the batch, features
    // q*P .. q*P + P-1
    const uint32_t rl = PAIRED ? (uint32_t)lane >> 1 : (uint32_t)lane % (uint32_t)RPB;
    const uint32_t q = PAIRED ? (uint32_t)lane & 1u : (uint32_t)lane / (uint32_t)RPB;
    const uint32_t byte_off = q * (uint32_t)P;
    // x: the lane's rotation; at step s it adds byte (feature) x ^ s of its P
    const uint32_t x = PAIRED ? rl & (uint32_t)(P - 1) : (uint32_t)lane & (uint32_t)(P - 1);
    const uint32_t m = x >> 2;
    const uint32_t cx = P == 32 ? (m >> 2) : 0u;
    const bool b0 = (m & 1u) != 0, b1 = (m & 2u) != 0;
    // W = 64: feature q*P + x sits in plane (q*P) >> 5, column ((q*P) & 31) + x;
    // W = 32: plane 0, column q*P + x (both half-waves share it)
    const uint32_t colbase =
        W == 64 ? (((q * (uint32_t)P) >> 5) << 16) | ((((q * (uint32_t)P) & 31u) + rl) << 3)
        : W == 32 ? ((q * (uint32_t)P + x) << 3)
                  : (((uint32_t)(lane >> 5) << 16) | (((uint32_t)lane & 31u) << 3));
    uint32_t colw[HIST_COLW_TABLE ? P : 1];
    if constexpr (HIST_COLW_TABLE) {
#pragma unroll
        for (int s = 0; s < P; ++s) colw[s] = colbase ^ ((uint32_t)s << 3);
    }
    uint32_t sel[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
        sel[t] = 0x0C020000u | ((4u + ((x & 3u) ^ (uint32_t)t)) << 8);
    // extra step j: plane 1, column (lane & 31) ^ j (paired: one step, column
    // 16q + x)
    const uint32_t cwx0 = PAIRED ? 0x10000u | ((q * 16u + x) << 3)
                                 : 0x10000u | (((uint32_t)lane & 31u) << 3);
    const uint32_t cwx1 = cwx0 ^ 8u;
    char *lds = reinterpret_cast<char *>(hist_lds);
    const uint32_t stride = nwaves * RPB;
    const uint32_t nitems = ctl->num_items;
    // Items are chunk-major (the tiles of one row chunk are adjacent).  With
    // workgroups dispatched round-robin over 8 XCDs (block b on XCD b % 8),
    // XCD x takes the contiguous items x*G/8 .. (x+1)*G/8 - 1 of each round of
    // G, so the tile items of a chunk read the same row lines through one L2
    // (always at 2 tiles per chunk; at 3, all but the chunks split by a range
    // boundary).
    uint32_t slot = blockIdx.x;
    if ((gridDim.x & 7u) == 0) slot = (blockIdx.x & 7u) * (gridDim.x >> 3) + (blockIdx.x >> 3);
    for (uint32_t it = slot; it < nitems; it += gridDim.x) {
        const HistItem item = items[it];
        const uint32_t cnt = item.count;            // >= 1
        const uint32_t last = cnt - 1;
        for (int k = tid; k < LDS_BYTES / 16; k += HIST_THREADS)
            reinterpret_cast<uint4 *>(hist_lds)[k] = make_uint4(0, 0, 0, 0);
        __syncthreads();
        const uint8_t *tile = tiled + (size_t)item.tile * (size_t)lay.tile_step + byte_off;
        const size_t row_bytes =
            (size_t)((int32_t)item.tile == lay.last_tile ? lay.last_stride : lay.stride);
        const Entry *ent = order + item.start;
        const uint32_t *ent_q = reinterpret_cast<const uint32_t *>(order) + item.start;
        // the item's extras: count, first, and the per-lane byte selectors
        const int32_t ne = XTRA ? tile_extra_count(sh, (int32_t)item.tile) : 0;
        const int32_t xf = XTRA ? tile_extra_first(sh, (int32_t)item.tile) : 0;
        const uint32_t *xsrc = reinterpret_cast<const uint32_t *>(
            tiled + lay.x_off + (size_t)(xf & ~3));
        const size_t xs4 = (size_t)(lay.x_stride >> 2);
        const uint32_t xb = (uint32_t)(xf & 3);
        // paired: lane q adds extra q (byte 3 at most: the dword's last)
        const uint32_t e0 = PAIRED ? q : ne == 2 ? ((uint32_t)lane & 1u) : 0u;
        const uint32_t selx0 = 0x0C020000u | ((4u + min(xb + e0, 3u)) << 8);
        const uint32_t selx1 = 0x0C020000u | ((4u + xb + (e0 ^ 1u)) << 8);
        // entry j of the item (IMPLICIT: row start + j with its packed word)
        auto entry = [&](uint32_t j) {
            if constexpr (IMPLICIT) return Entry{item.start + j, ent_q[j]};
            else return ent[j];
        };
        auto load_x = [&](uint32_t row) -> uint32_t {
            if constexpr (XTRA) return ne ? xsrc[(size_t)row * xs4] : 0u;
            else return 0u;
        };
        const uint32_t g0 = (uint32_t)wave * RPB;
        // loads past the item's end read its last entry (in bounds); their
        // rows are given value 0 when processed
        Entry er[ER];
        RowRaw<P> dr[DR];
        uint32_t xr[XTRA ? DR : 1];
        // Prologue in the main loop's issue order: the entries the first
        // data loads need, then each data batch followed by the entry ER - DR
        // batches after it.  Memory waits count loads in issue order, so at
        // the loop head both paths then leave the same loads outstanding and
        // the compiler's merged wait counts are the steady state's (issued
        // entries-first, the first batches of every round waited with data
        // only one or two batches ahead: deep levels 1% slower).
#pragma unroll
        for (int k = 0; k < ER - DR; ++k) er[k] = entry(min(g0 + (uint32_t)k * stride + rl, last));
#pragma unroll
        for (int k = 0; k < DR; ++k) {
            dr[k] = load_row_raw<P>(tile + (size_t)er[k].row * row_bytes, cx);
            if constexpr (XTRA) xr[k] = load_x(er[k].row);
            er[ER - DR + k] = entry(min(g0 + (uint32_t)(ER - DR + k) * stride + rl, last));
            __builtin_amdgcn_sched_barrier(0);       // keep this issue order
        }
        auto process = [&](uint32_t g, const Entry &e, const RowRaw<P> &raw, uint32_t x) {
            // rows past the item's end carry value 0
            const uint32_t ghq = g + rl < cnt ? e.ghq : 0u;
            const int32_t qg = (int32_t)(int16_t)(uint16_t)(ghq >> 16);
            const unsigned long long v = (unsigned long long)((int64_t)qg * (1ll << HIST_QH_BITS)) +
                                         (unsigned long long)(ghq & 0x7Fu);
            const RowRaw<P> cur = permute_dwords<P>(raw, b0, b1);
#pragma unroll
            for (int s = 0; s < P; ++s) {
                const uint32_t cw = HIST_COLW_TABLE ? colw[HIST_COLW_TABLE ? s : 0]
                                                    : colbase ^ ((uint32_t)s << 3);
                const uint32_t addr = __builtin_amdgcn_perm(cur.d[s >> 2], cw, sel[s & 3]);
                atomicAdd(reinterpret_cast<unsigned long long *>(lds + addr), v);
            }
            if constexpr (XTRA) {
                if (ne >= 1) {                       // uniform per item
                    const uint32_t addr = __builtin_amdgcn_perm(x, cwx0, selx0);
                    atomicAdd(reinterpret_cast<unsigned long long *>(lds + addr), v);
                }
                if (!PAIRED && ne >= 2) {
                    const uint32_t addr = __builtin_amdgcn_perm(x, cwx1, selx1);
                    atomicAdd(reinterpret_cast<unsigned long long *>(lds + addr), v);
                }
            }
        };
        // main rounds: all ER batches exist, no exits inside the round, so the
        // refill loads stay where they are issued
        uint32_t base = g0;
        for (; base + (uint32_t)(ER - 1) * stride < cnt; base += (uint32_t)ER * stride) {
#pragma unroll
            for (int k = 0; k < ER; ++k) {
                const uint32_t g = base + (uint32_t)k * stride;
                process(g, er[k], dr[k % DR], XTRA ? xr[XTRA ? k % DR : 0] : 0u);
                // refill: data for batch +DR (its entry is already held), entry for batch +ER
                dr[k % DR] = load_row_raw<P>(tile + (size_t)er[(k + DR) % ER].row * row_bytes, cx);
                if constexpr (XTRA) xr[k % DR] = load_x(er[(k + DR) % ER].row);
                er[k] = entry(min(g + (uint32_t)ER * stride + rl, last));
            }
        }
        // tail: fewer than ER batches left; entries are held, data up to DR ahead
#pragma unroll
        for (int k = 0; k < ER; ++k) {
            const uint32_t g = base + (uint32_t)k * stride;
            if (g >= cnt) break;                     // uniform per wavefront
            process(g, er[k], dr[k % DR], XTRA ? xr[XTRA ? k % DR : 0] : 0u);
            if (k + DR < ER) {
                dr[k % DR] = load_row_raw<P>(tile + (size_t)er[(k + DR) % ER].row * row_bytes, cx);
                if constexpr (XTRA) xr[k % DR] = load_x(er[(k + DR) % ER].row);
            }
        }
        __syncthreads();
        // flush to the item's partial, layout [nb][PW]; padding columns (past
        // the last feature, or extras the tile does not carry) are neither
        // written nor read
        uint64_t *out = partials + (size_t)it * (size_t)(nb * PW);
        const int wreal = min(W, cols - (int)item.tile * W);
        for (int k = tid; k < nb * PW; k += HIST_THREADS) {
            const int b = k / PW, f = k % PW;
            uint64_t acc = 0;
            if (f < W) {
                if (f >= wreal) continue;
                if constexpr (W == 64) {
                    acc = hist_lds[(f >> 5) * 8192 + b * 32 + (f & 31)];
                } else if constexpr (W == 32) {
                    acc = hist_lds[b * 32 + f];
                } else {
                    constexpr int CPP = 32 / W;      // copies per plane
#pragma unroll
                    for (int c = 0; c < 64 / W; ++c)
                        acc += hist_lds[(c / CPP) * 8192 + b * 32 + (c % CPP) * W + f];
                }
            } else if constexpr (XTRA) {
                // extra e: plane 1, columns c with c % ne == e (paired: 16e .. 16e+15)
                const int e = f - W;
                if (e >= ne) continue;
                if constexpr (PAIRED) {
                    const uint64_t *src = hist_lds + 8192 + b * 32 + 16 * e;
#pragma unroll
                    for (int c = 0; c < 16; ++c) acc += src[c];
                } else {
                    for (int c = e; c < 32; c += ne) acc += hist_lds[8192 + b * 32 + c];
                }
            } else {
                continue;                            // no extras without plane 1
            }
            __builtin_nontemporal_store(acc, &out[k]);   // read once, by k_reduce
        }
        __syncthreads();
    }
}


HistLayout gather_layout(const Shape &sh) {
    const int32_t row = sh.num_tiles * sh.tile_w;
    return HistLayout{(int64_t)sh.tile_w, row, row, sh.num_tiles - 1, row,
                      (int64_t)sh.hist_tiles * sh.tile_w};
}

// Bytes of the extras plane per row: the extras rounded up to a dword.
static int32_t extras_pitch(const Shape &sh) { return (sh.extras + 3) / 4 * 4; }

bool has_planar_layout(const Shape &sh) {
    if (sh.tile_w == 32) return sh.extras > 0;
    if (sh.tile_w != 64 || sh.num_tiles < 2) return false;
    const int32_t last_feats = sh.cols - (sh.num_tiles - 1) * 64;
    return (last_feats + 15) / 16 * 16 < 64;         // else the copy saves nothing
}

HistLayout planar_layout(const Shape &sh) {
    if (sh.tile_w == 32)
        return HistLayout{sh.rows * 32, 32, 32, sh.num_tiles - 1, extras_pitch(sh),
                          (int64_t)sh.hist_tiles * sh.rows * 32};
    const int32_t last_feats = sh.cols - (sh.num_tiles - 1) * 64;
    return HistLayout{sh.rows * 64, 64, (last_feats + 15) / 16 * 16, sh.num_tiles - 1, 0, 0};
}

size_t planar_bytes(const Shape &sh) {
    const HistLayout l = planar_layout(sh);
    if (sh.tile_w == 32) return (size_t)l.x_off + (size_t)sh.rows * (size_t)l.x_stride + 64;
    return (size_t)l.last_tile * (size_t)l.tile_step + (size_t)sh.rows * (size_t)l.last_stride + 64;
}

hipError_t launch_hist(hipStream_t s, const Shape &sh, const uint8_t *tiled, const Entry *order,
                       const HistItem *items, const TreeCtl *ctl, uint64_t *partials, int grid,
                       const HistLayout *layout, hipEvent_t start, hipEvent_t stop,
                       bool implicit_rows) {
    const HistLayout lay = layout ? *layout : gather_layout(sh);
    if (sh.hist_tiles < 1 || sh.part_w < sh.tile_w ||
        (sh.extras > 0 && (sh.tile_w != 32 || sh.hist_tiles != sh.num_tiles - 1)))
        return hipErrorInvalidValue;
    if (layout) {
        // the planar copy, exactly as planar_layout lays it out
        const HistLayout p = planar_layout(sh);
        if (!has_planar_layout(sh) || lay.tile_step != p.tile_step || lay.stride != p.stride ||
            lay.last_stride != p.last_stride || lay.last_tile != p.last_tile ||
            lay.x_stride != p.x_stride || lay.x_off != p.x_off)
            return hipErrorInvalidValue;
    }
    switch (sh.tile_w) {
#define MBK_COMMA ,
#define MBK_HIST_LAUNCH(KERN)                                                                    \
    {                                                                                            \
        auto *kern = &KERN;                                                                      \
        if (start || stop)                                                                       \
            hipExtLaunchKernelGGL(kern, dim3(grid), dim3(HIST_THREADS), 0, s, start, stop, 0,    \
                                  tiled, order, items, ctl, partials, lay, sh);                  \
        else                                                                                     \
            hipLaunchKernelGGL(kern, dim3(grid), dim3(HIST_THREADS), 0, s, tiled, order, items,  \
                               ctl, partials, lay, sh);                                          \
    }
#define MBK_HIST_CASE(WW, LL)                                                                    \
        if (implicit_rows) MBK_HIST_LAUNCH(k_hist<WW MBK_COMMA LL MBK_COMMA true>)              \
        else MBK_HIST_LAUNCH(k_hist<WW MBK_COMMA LL MBK_COMMA false>)                            \
        break;
    case 8: MBK_HIST_CASE(8, 1)
    case 16: MBK_HIST_CASE(16, 1)
    case 32:
        // gathered rows of an ordered level: two lanes per row (one 16-B load
        // each; HIGGS-like 10M x 28: levels 1-5 together -3%); streamed rows
        // (planar copy, or the implicit root, 3% faster): one row per lane
        if (layout || implicit_rows) {
            MBK_HIST_CASE(32, 1)
        } else {
            MBK_HIST_LAUNCH(k_hist<32 MBK_COMMA 2 MBK_COMMA false>)
            break;
        }
    case 64:
        if (layout) { MBK_HIST_CASE(64, 2) }         // planar rows: contiguous, two lanes per row
        else { MBK_HIST_CASE(64, 4) }                // gathered rows: one load per row and tile
#undef MBK_HIST_CASE
#undef MBK_HIST_LAUNCH
#undef MBK_COMMA
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t hist_lds_size() { return (size_t)HIST_LDS_BYTES; }

// Planar copy of the gather layout for the root pass (planar_layout): 16-B
// chunk j of row r (j < 4 * (T - 1) + last_stride / 16, i.e. every feature and
// its zero padding up to a 16-B multiple) goes to tile j / 4's plane.  One
// thread per chunk of the output.
__global__ __launch_bounds__(256) void k_planar_rows(const uint8_t *__restrict__ tiled,
                                                     int64_t rows, int32_t row_bytes,
                                                     HistLayout lay, uint8_t *__restrict__ out) {
    const int32_t full = 4 * lay.last_tile, per_row = full + lay.last_stride / 16;
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= rows * per_row) return;
    const int64_t r = k / per_row;
    const int32_t j = (int32_t)(k - r * per_row);
    const int64_t dst = j < full
        ? (int64_t)(j >> 2) * lay.tile_step + r * 64 + (j & 3) * 16
        : (int64_t)lay.last_tile * lay.tile_step + r * lay.last_stride + (j - full) * 16;
    *reinterpret_cast<uint4 *>(out + dst) =
        *reinterpret_cast<const uint4 *>(tiled + r * row_bytes + (int64_t)j * 16);
}

// The 32-wide form with extras: item j < 2 (T - 1) of row r copies 16-B chunk
// j to tile j / 2's plane, item 2 (T - 1) copies the row's extra bytes (from
// the last tile, in dwords) to the extras plane.
__global__ __launch_bounds__(256) void k_planar_rows32(const uint8_t *__restrict__ tiled,
                                                       int64_t rows, int32_t row_bytes,
                                                       int32_t main_tiles, HistLayout lay,
                                                       uint8_t *__restrict__ out) {
    const int32_t per_row = 2 * main_tiles + 1;
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= rows * per_row) return;
    const int64_t r = k / per_row;
    const int32_t j = (int32_t)(k - r * per_row);
    const uint8_t *src = tiled + r * row_bytes;
    if (j < 2 * main_tiles) {
        *reinterpret_cast<uint4 *>(out + (int64_t)(j >> 1) * lay.tile_step + r * 32 + (j & 1) * 16) =
            *reinterpret_cast<const uint4 *>(src + (int64_t)j * 16);
        return;
    }
    const uint32_t *xs = reinterpret_cast<const uint32_t *>(src + (int64_t)main_tiles * 32);
    uint32_t *xd = reinterpret_cast<uint32_t *>(out + lay.x_off + r * lay.x_stride);
    for (int32_t w = 0; w < lay.x_stride / 4; ++w) xd[w] = xs[w];
}

hipError_t launch_planar_rows(hipStream_t s, const Shape &sh, const uint8_t *tiled,
                              int32_t row_bytes, uint8_t *out) {
    if (!has_planar_layout(sh)) return hipErrorInvalidValue;
    const HistLayout lay = planar_layout(sh);
    // the source rows must hold every byte a copy reads (feature f at byte f)
    const int32_t need = sh.tile_w == 32 ? sh.hist_tiles * 32 + lay.x_stride
                                         : sh.num_tiles * sh.tile_w;
    if (row_bytes < need || row_bytes % 16 != 0) return hipErrorInvalidValue;
    if (sh.tile_w == 32) {
        const int64_t n = sh.rows * (2 * sh.hist_tiles + 1);
        if (n <= 0) return hipSuccess;
        hipLaunchKernelGGL(k_planar_rows32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           tiled, sh.rows, row_bytes, sh.hist_tiles, lay, out);
        return hipGetLastError();
    }
    const int64_t n = sh.rows * (4 * lay.last_tile + lay.last_stride / 16);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_planar_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, tiled,
                       sh.rows, row_bytes, lay, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// partial reduction + sibling subtraction (subtract_histograms, :313-326):
// one thread per (pair, tile, bin, feature), fully coalesced; histograms are
// stored [node][bin][feature][g,h] as exact int64.
// ---------------------------------------------------------------------------

// A block of 256 threads covers 256 / S (bin, feature) cells of one (pair,
// tile); its S slices of threads split that tile's chunks.  Levels with 16 or
// more pairs (few chunks each) run with S = 1, the others with S = 4.
template <int S>
__global__ __launch_bounds__(256) void k_reduce(Shape sh, const Pair *__restrict__ pairs,
                                                const uint64_t *__restrict__ partials,
                                                const int64_t *__restrict__ hist_prev,
                                                int64_t *__restrict__ hist_cur, const TreeCtl *ctl,
                                                uint32_t blocks_per_tile, int derive,
                                                uint64_t *keys, uint64_t *cursors,
                                                uint32_t nzero) {
    constexpr int CELLS = 256 / S;
    __shared__ int64_t red[S > 1 ? S : 1][CELLS][2];
    if (blockIdx.x == 0) {
        // the level's split keys (maxima from the split search next) and
        // partition cursors (used by the next partition) start from zero
        for (uint32_t l = threadIdx.x; l < nzero; l += blockDim.x) {
            if (keys) keys[(size_t)l * KEY_STRIDE] = 0;
            if (cursors) cursors[(size_t)l * CURSOR_STRIDE] = 0;
        }
    }
    const int PW = sh.part_w, nb = sh.num_bins, F = sh.cols, T = sh.hist_tiles;
    const uint32_t bpt = blockIdx.x % blocks_per_tile;
    const uint32_t rest = blockIdx.x / blocks_per_tile;
    const int tile = (int)(rest % (uint32_t)T);
    const uint32_t pair_idx = rest / (uint32_t)T;
    if (pair_idx >= ctl->num_pairs) return;          // uniform per block
    const int kk = threadIdx.x % CELLS, slice = threadIdx.x / CELLS;
    const int k = (int)bpt * CELLS + kk;             // (bin, column) index in the item partial
    const Pair pr = pairs[pair_idx];
    // the column's feature (main or extra), -1 for padding: those hold no partials
    const int f = k < nb * PW ? partial_feature(sh, tile, k % PW) : -1;
    int64_t g = 0, h = 0;
    if (f >= 0) {
        const size_t stride = (size_t)(nb * PW);
        const size_t cstride = (size_t)T * stride;   // between chunks of one (pair, tile)
        const uint64_t *src = partials + ((size_t)pr.item_first + (size_t)tile) * stride + k;
        constexpr uint64_t HMASK = (1ull << HIST_QH_BITS) - 1;
        // four chunks per step, their loads in flight together (integer sums:
        // the order does not matter); partials are read once, so their loads
        // and the histogram kernel's stores are nontemporal
        uint32_t c = (uint32_t)slice;
        for (; c + 3 * S < pr.nchunks; c += 4 * S) {
            uint64_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[j] = __builtin_nontemporal_load(&src[(size_t)(c + j * S) * cstride]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                g += (int64_t)w[j] >> HIST_QH_BITS;
                h += (int64_t)(w[j] & HMASK);
            }
        }
        for (; c < pr.nchunks; c += S) {
            const uint64_t w1 = __builtin_nontemporal_load(&src[(size_t)c * cstride]);
            g += (int64_t)w1 >> HIST_QH_BITS;
            h += (int64_t)(w1 & HMASK);
        }
    }
    if constexpr (S > 1) {
        red[slice][kk][0] = g;
        red[slice][kk][1] = h;
        __syncthreads();
        if (slice != 0) return;
        for (int s2 = 1; s2 < S; ++s2) { g += red[s2][kk][0]; h += red[s2][kk][1]; }
    }
    if (f < 0) return;
    const int b = k / PW;
    int64_t *hb = hist_cur + (((size_t)pr.built * nb + b) * F + f) * 2;
    hb[0] = g;
    hb[1] = h;
    if (derive && pr.derived != NONE) {
        const int64_t *hp = hist_prev + (((size_t)pr.parent * nb + b) * F + f) * 2;
        int64_t *hd = hist_cur + (((size_t)pr.derived * nb + b) * F + f) * 2;
        hd[0] = hp[0] - g;
        hd[1] = hp[1] - h;
    }
}

hipError_t launch_reduce(hipStream_t s, const Shape &sh, const Pair *pairs, uint32_t max_pairs,
                         const uint64_t *partials, const int64_t *hist_prev, int64_t *hist_cur,
                         const TreeCtl *ctl, bool derive, uint64_t *keys, uint64_t *cursors,
                         uint32_t nzero) {
    const uint32_t cells = (uint32_t)(sh.num_bins * sh.part_w);
    const int dv = derive ? 1 : 0;
    if (!keys && !cursors) nzero = 0;
    if (max_pairs >= 32) {                           // measured: S = 4 is faster below
        const uint32_t bpt = (cells + 255) / 256;
        hipLaunchKernelGGL(k_reduce<1>, dim3(max_pairs * (uint32_t)sh.hist_tiles * bpt), dim3(256),
                           0, s, sh, pairs, partials, hist_prev, hist_cur, ctl, bpt, dv, keys,
                           cursors, nzero);
    } else {
        const uint32_t bpt = (cells + 63) / 64;
        hipLaunchKernelGGL(k_reduce<4>, dim3(max_pairs * (uint32_t)sh.hist_tiles * bpt), dim3(256),
                           0, s, sh, pairs, partials, hist_prev, hist_cur, ctl, bpt, dv, keys,
                           cursors, nzero);
    }
    return hipGetLastError();
}

// Sibling by subtraction on its own (subtract_histograms, Shaders.swift:313-326):
// derived = parent - built for every pair of the level, exact int64, one
// thread per (pair, bin, feature, channel).
__global__ __launch_bounds__(256) void k_subtract(Shape sh, const Pair *__restrict__ pairs,
                                                  const int64_t *__restrict__ hist_prev,
                                                  int64_t *__restrict__ hist_cur,
                                                  const TreeCtl *ctl, uint32_t blocks_per_pair) {
    const uint32_t p = blockIdx.x / blocks_per_pair;
    if (p >= ctl->num_pairs) return;                 // uniform per block
    const Pair pr = pairs[p];
    if (pr.derived == NONE) return;
    const size_t cells = (size_t)sh.num_bins * (size_t)sh.cols * 2;
    const size_t k = (size_t)(blockIdx.x % blocks_per_pair) * 256 + threadIdx.x;
    if (k >= cells) return;
    hist_cur[(size_t)pr.derived * cells + k] =
        hist_prev[(size_t)pr.parent * cells + k] - hist_cur[(size_t)pr.built * cells + k];
}

hipError_t launch_subtract(hipStream_t s, const Shape &sh, const Pair *pairs, uint32_t max_pairs,
                           const int64_t *hist_prev, int64_t *hist_cur, const TreeCtl *ctl) {
    const size_t cells = (size_t)sh.num_bins * (size_t)sh.cols * 2;
    const uint32_t bpp = (uint32_t)((cells + 255) / 256);
    if (max_pairs == 0) return hipSuccess;
    hipLaunchKernelGGL(k_subtract, dim3(max_pairs * bpp), dim3(256), 0, s, sh, pairs, hist_prev,
                       hist_cur, ctl, bpp);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// split search: one wavefront per (sibling pair, feature)
// ---------------------------------------------------------------------------

// LDS visibility between the lanes of one wavefront (each wave owns its
// scratch, so no workgroup barrier is needed).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct CatScratch {
    float key[256];
    int64_t sg[256];
    int64_t sh[256];
    uint32_t mask[8];
};

// Best split of one node's feature histogram held as 4 consecutive bins per
// lane (bins 4*lane .. 4*lane+3).  Mirrors find_splits (Shaders.swift:396-463)
// with exact integer prefix sums.  Writes the result through dst (one lane)
// and returns its gain in every lane (-inf: no valid split).
__device__ float node_split(const int64_t (&hg)[4], const int64_t (&hh)[4], int32_t nb,
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
            return -INFINITY;
        } else if (ws == best_seq && best_gain == wg) {
            SplitResult r = {};
            r.gain = best_gain; r.bin = best_bin; r.gl = best_gl; r.hl = best_hl;
            r.flags = best_flags; r.gl_int = best_gli; r.hl_int = best_hli;
            *dst = r;
        }
        return wg;
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
    wave_lds_sync();
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
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ne[j]) { cs->sg[rank[j]] = hg[j]; cs->sh[rank[j]] = hh[j]; }
    wave_lds_sync();
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
        return -INFINITY;
    }
    const int k = ws + 1;                            // left subset size
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ne[j] && rank[j] < k) atomicOr(&cs->mask[(b0 + j) >> 5], 1u << ((b0 + j) & 31));
    wave_lds_sync();
    if (ws == best_seq && best_gain == wg) {
        SplitResult r = {};
        r.gain = best_gain; r.bin = best_bin; r.gl = best_gl; r.hl = best_hl;
        r.flags = best_flags; r.gl_int = best_gli; r.hl_int = best_hli;
#pragma unroll
        for (int w = 0; w < 8; ++w) r.mask[w] = cs->mask[w];
        *dst = r;
    }
    return wg;
}

// One workgroup per (sibling pair, 4 features), one wavefront per (side,
// feature): both sides' histogram rows [bin][f0 .. f0+3] (64 contiguous bytes
// per bin) are staged through LDS together, eight independent loads per
// thread, then wavefront (side, w) searches feature f0 + w of that side's node
// (its 256 bins, 4 per lane).  The two sides' searches run at once.
constexpr int SPLIT_FEATS = 4;
constexpr int SPLIT_WAVES = 2 * SPLIT_FEATS;
constexpr int SPLIT_THREADS = SPLIT_WAVES * 64;
constexpr int SPLIT_ROW = 2 * SPLIT_FEATS;           // words per bin and side
constexpr int SPLIT_STAGE_PER_THREAD = 2 * 256 * SPLIT_ROW / SPLIT_THREADS;
constexpr size_t SPLIT_STAGE_BYTES = (size_t)2 * 256 * SPLIT_ROW * sizeof(int64_t);
constexpr size_t SPLIT_LDS_BYTES = SPLIT_STAGE_BYTES > SPLIT_WAVES * sizeof(CatScratch)
                                       ? SPLIT_STAGE_BYTES
                                       : SPLIT_WAVES * sizeof(CatScratch);
static_assert(2 * 256 * SPLIT_ROW % SPLIT_THREADS == 0, "whole stage words per thread");

__global__ __launch_bounds__(SPLIT_THREADS) void k_split(Shape sh, SplitParams sp,
                                                         const Pair *__restrict__ pairs,
                                                         const int64_t *__restrict__ hist_cur,
                                                         const uint8_t *__restrict__ is_cat,
                                                         const int8_t *__restrict__ monotone,
                                                         const uint8_t *__restrict__ feat_mask,
                                                         const TreeCtl *ctl, const uint32_t *count,
                                                         int64_t *node_g, int64_t *node_h,
                                                         uint32_t level_start,
                                                         SplitResult *__restrict__ results,
                                                         uint64_t *keys) {
    __shared__ __align__(16) unsigned char split_lds[SPLIT_LDS_BYTES];
    int64_t *stage = reinterpret_cast<int64_t *>(split_lds);      // [side][bin][SPLIT_ROW]
    CatScratch *cs_all = reinterpret_cast<CatScratch *>(split_lds);
    const int F = sh.cols, nb = sh.num_bins;
    const uint32_t groups = (uint32_t)((F + SPLIT_FEATS - 1) / SPLIT_FEATS);
    const uint32_t pair_idx = blockIdx.x / groups;
    const int f0 = (int)(blockIdx.x % groups) * SPLIT_FEATS;
    if (pair_idx >= ctl->num_pairs) return;          // uniform per block
    const int nf = min(SPLIT_FEATS, F - f0);
    const Pair pr = pairs[pair_idx];
    const int tid = threadIdx.x, lane = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int side = w / SPLIT_FEATS, fw = w % SPLIT_FEATS;
    const int f = f0 + fw;
    const uint32_t local = side == 0 ? pr.built : pr.derived;
    const bool active = fw < nf && local != NONE;
    __shared__ unsigned long long s_key[2];          // the workgroup's best key per side
    if (tid < 2) s_key[tid] = 0;
    // stage both sides' rows (a side without a node stages zeros)
    const int row = 2 * nf;
    int64_t v[SPLIT_STAGE_PER_THREAD];
#pragma unroll
    for (int k = 0; k < SPLIT_STAGE_PER_THREAD; ++k) {
        const int idx = tid + k * SPLIT_THREADS;
        const int sd = idx / (256 * SPLIT_ROW), rem = idx - sd * (256 * SPLIT_ROW);
        const int b = rem / row, r = rem - b * row;
        const uint32_t node = sd == 0 ? pr.built : pr.derived;
        v[k] = (b < nb && node != NONE)
                   ? hist_cur[(((size_t)node * nb + b) * F + f0) * 2 + r]
                   : 0;
    }
#pragma unroll
    for (int k = 0; k < SPLIT_STAGE_PER_THREAD; ++k) {
        const int idx = tid + k * SPLIT_THREADS;
        const int sd = idx / (256 * SPLIT_ROW), rem = idx - sd * (256 * SPLIT_ROW);
        const int b = rem / row, r = rem - b * row;
        if (b < nb) stage[((size_t)sd * 256 + b) * SPLIT_ROW + r] = v[k];
    }
    __syncthreads();
    int64_t hg[4], hh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        hg[j] = 0; hh[j] = 0;
        if (active && b < nb) {
            hg[j] = stage[((size_t)side * 256 + b) * SPLIT_ROW + 2 * fw];
            hh[j] = stage[((size_t)side * 256 + b) * SPLIT_ROW + 2 * fw + 1];
        }
    }
    __syncthreads();                                 // the stage becomes split scratch
    if (active) {                                    // uniform per wavefront
        const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
        const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;
        const bool cat = is_cat[f] != 0;
        const int cst = cat ? 0 : (int)monotone[f];
        const bool allowed = feat_mask[f] != 0;
        const uint32_t abs_n = level_start + local;
        if (f == 0) {
            const int64_t G = wave_sum(hg[0] + hg[1] + hg[2] + hg[3]);
            const int64_t H = wave_sum(hh[0] + hh[1] + hh[2] + hh[3]);
            if (lane == 0) { node_g[abs_n] = G; node_h[abs_n] = H; }
        }
        SplitResult *dst = results + (size_t)local * F + f;
        if (allowed && count[abs_n] >= 1) {
            const float g = node_split(hg, hh, nb, cat, cst, g_inv, h_inv, sp, &cs_all[w], dst);
            const uint64_t k = keys ? split_key(g, f) : 0;
            if (lane == 0 && k) atomicMax(&s_key[side], (unsigned long long)k);
        } else if (lane == 0) {
            SplitResult r = {};
            r.gain = -INFINITY;
            *dst = r;
        }
    }
    if (keys) {                                      // uniform
        // the node's argmax over features, for the next partition's
        // decisions: one global maximum per workgroup and side (each node's
        // key on its own 128-B line; same-line atomics serialize)
        __syncthreads();
        if (tid < 2) {
            const uint32_t node = tid == 0 ? pr.built : pr.derived;
            if (node != NONE && s_key[tid])
                atomicMax(reinterpret_cast<unsigned long long *>(&keys[(size_t)node * KEY_STRIDE]),
                          s_key[tid]);
        }
    }
}

hipError_t launch_split(hipStream_t s, const Shape &sh, const SplitParams &sp, const Pair *pairs,
                        uint32_t max_pairs, const uint64_t *partials, const int64_t *hist_prev,
                        int64_t *hist_cur, const uint8_t *is_cat, const int8_t *monotone,
                        const uint8_t *feat_mask, const TreeCtl *ctl, const uint32_t *count,
                        int64_t *node_g, int64_t *node_h, uint32_t level_start,
                        SplitResult *results, uint64_t *keys, uint64_t *cursors) {
    if (sh.num_bins > 256) return hipErrorInvalidValue;
    // level_start = 2^d - 1: the level holds level_start + 1 nodes
    hipError_t e = launch_reduce(s, sh, pairs, max_pairs, partials, hist_prev, hist_cur, ctl, true,
                                 keys, cursors, level_start + 1);
    if (e != hipSuccess) return e;
    return launch_find_splits(s, sh, sp, pairs, max_pairs, hist_cur, is_cat, monotone, feat_mask,
                              ctl, count, node_g, node_h, level_start, results, keys);
}

hipError_t launch_find_splits(hipStream_t s, const Shape &sh, const SplitParams &sp,
                              const Pair *pairs, uint32_t max_pairs, const int64_t *hist_cur,
                              const uint8_t *is_cat, const int8_t *monotone,
                              const uint8_t *feat_mask, const TreeCtl *ctl, const uint32_t *count,
                              int64_t *node_g, int64_t *node_h, uint32_t level_start,
                              SplitResult *results, uint64_t *keys) {
    if (sh.num_bins > 256) return hipErrorInvalidValue;
    const uint32_t groups = (uint32_t)((sh.cols + SPLIT_FEATS - 1) / SPLIT_FEATS);
    hipLaunchKernelGGL(k_split, dim3(max_pairs * groups), dim3(SPLIT_THREADS), 0, s, sh, sp, pairs,
                       hist_cur, is_cat, monotone, feat_mask, ctl, count, node_g, node_h,
                       level_start, results, keys);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decisions: one wavefront per node (decide_splits phase 1, :1386-1451)
// ---------------------------------------------------------------------------

__device__ void decide_apply(const SplitParams &sp, int F, uint32_t n, uint32_t local, int bf,
                             float bg, const SplitResult *__restrict__ results, int64_t Gt,
                             int64_t Ht, float2 pb, uint32_t mgb, uint32_t mhb, int64_t *node_g,
                             int64_t *node_h, float2 *bounds, const int8_t *monotone,
                             const TreeOut &out);

// decide_splits for node `local` of level la (Shaders.swift:1342-1452), run by
// one wavefront: argmax over features, then the node's split or leaf, the
// children's sums and monotone bounds; also zeroes the node's partition
// cursor for the level's partition.
__device__ void decide_node(const Shape &sh, const SplitParams &sp, const LevelArgs &la,
                            uint32_t local, const SplitResult *__restrict__ results,
                            const uint32_t *count, int64_t *node_g, int64_t *node_h,
                            float2 *bounds, const int8_t *monotone, const TreeCtl *ctl,
                            uint64_t *cursors, const TreeOut &out) {
    const uint32_t n = la.level_start + local;
    const int lane = lane_id();
    const int F = sh.cols;
    // the partition of this level starts from zeroed cursors
    if (lane == 0) cursors[(size_t)local * CURSOR_STRIDE] = 0;
    if (count[n] < 1) {
        if (lane == 0) {
            NodeSplit leaf = {-1, 0, 0};
            out.split[n] = leaf;
            out.leaf[n] = 0.0f;
            out.gain[n] = 0.0f;
        }
        return;
    }
    // the node's sums and bounds load while the feature argmax runs
    const uint32_t mgb = ctl->max_gh[0], mhb = ctl->max_gh[1];
    const int64_t Gt = node_g[n], Ht = node_h[n];
    const float2 pb = bounds[n];
    float bg = -INFINITY;
    int bf = 0x7FFFFFFF;
    for (int f = lane; f < F; f += 64) {
        const float g = results[(size_t)local * F + f].gain;
        if (g > bg) { bg = g; bf = f; }               // f ascending within the lane
    }
    wave_argmax(bg, bf);
    if (lane != 0) return;
    decide_apply(sp, F, n, local, bf == 0x7FFFFFFF ? -1 : bf, bg, results, Gt, Ht, pb, mgb, mhb,
                 node_g, node_h, bounds, monotone, out);
}

// decide_splits' outcome for node n (level-local `local`) once its best
// feature bf (-1: none) and gain bg are known, by one lane: the node's split
// or leaf, the children's sums and monotone bounds (Shaders.swift:1401-1451).
__device__ void decide_apply(const SplitParams &sp, int F, uint32_t n, uint32_t local, int bf,
                             float bg, const SplitResult *__restrict__ results, int64_t Gt,
                             int64_t Ht, float2 pb, uint32_t mgb, uint32_t mhb, int64_t *node_g,
                             int64_t *node_h, float2 *bounds, const int8_t *monotone,
                             const TreeOut &out) {
    const float g_inv = f32_from_bits(mgb) / 32767.0f;
    const float h_inv = f32_from_bits(mhb) / 127.0f;
    if (bf >= 0 && isfinite(bg) && bg > sp.min_split_gain) {
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
        const float G = (float)Gt * g_inv, H = (float)Ht * h_inv;
        out.leaf[n] = sp.learning_rate * clampf(-G / (H + sp.lambda), pb.x, pb.y);
    }
}

__global__ __launch_bounds__(64) void k_decide(Shape sh, SplitParams sp, LevelArgs la,
                                               const SplitResult *__restrict__ results,
                                               const uint32_t *count, int64_t *node_g,
                                               int64_t *node_h, float2 *bounds,
                                               const int8_t *monotone, const TreeCtl *ctl,
                                               uint64_t *cursors, TreeOut out) {
    decide_node(sh, sp, la, blockIdx.x, results, count, node_g, node_h, bounds, monotone, ctl,
                cursors, out);
}

hipError_t launch_decide(hipStream_t s, const Shape &sh, const SplitParams &sp,
                         const LevelArgs &la, const SplitResult *results, const uint32_t *count,
                         int64_t *node_g, int64_t *node_h, float2 *bounds,
                         const int8_t *monotone, const TreeCtl *ctl, uint64_t *cursors,
                         TreeOut out) {
    hipLaunchKernelGGL(k_decide, dim3(la.num_level), dim3(64), 0, s, sh, sp, la, results, count,
                       node_g, node_h, bounds, monotone, ctl, cursors, out);
    return hipGetLastError();
}

// Deepest level (final_leaves, Shaders.swift:1495-1511): leaf values of the
// children of split parents; their row counts are zeroed here and counted by
// the training walk (k_walk_count), and k_final_fixup then writes covers and
// sets empty leaves to 0.
// With counted != 0 the counts and covers already come from the partition
// (sampled trees) and empty leaves are 0 here.
__global__ void k_final_leaves(SplitParams sp, LevelArgs la, uint32_t *count,
                               const int64_t *node_g, const int64_t *node_h,
                               const float2 *bounds, const TreeCtl *ctl, TreeOut out,
                               int counted) {
    const uint32_t local = blockIdx.x * blockDim.x + threadIdx.x;
    if (local >= la.num_level) return;
    const uint32_t n = la.level_start + local;
    const uint32_t parent = (n - 1) >> 1;
    NodeSplit leaf = {-1, 0, 0};
    out.split[n] = leaf;
    out.gain[n] = 0.0f;
    bool filled;
    if (counted) {
        filled = count[n] >= 1;
    } else {
        count[n] = 0;
        filled = out.split[parent].feature >= 0 && count[parent] >= 1;
    }
    if (filled) {
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
                               uint32_t *count, const int64_t *node_g,
                               const int64_t *node_h, const float2 *bounds, const TreeCtl *ctl,
                               TreeOut out, bool counted) {
    hipLaunchKernelGGL(k_final_leaves, dim3((la.num_level + 255) / 256), dim3(256), 0, s, sp, la,
                       count, node_g, node_h, bounds, ctl, out, counted ? 1 : 0);
    return hipGetLastError();
}

__global__ void k_final_fixup(LevelArgs la, const uint32_t *count, TreeOut out,
                              int zero_empty) {
    const uint32_t local = blockIdx.x * blockDim.x + threadIdx.x;
    if (local >= la.num_level) return;
    final_fixup_node(la, count, out, zero_empty, local);
}

hipError_t launch_final_fixup(hipStream_t s, const LevelArgs &la, const uint32_t *count,
                              TreeOut out, bool zero_empty) {
    hipLaunchKernelGGL(k_final_fixup, dim3((la.num_level + 255) / 256), dim3(256), 0, s, la, count,
                       out, zero_empty ? 1 : 0);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// level planning (single workgroup): segment layout, sibling pairs, items
// ---------------------------------------------------------------------------

// Exclusive scan of v[0..n) in place by one block (a multiple of 64 threads,
// at most 1024); returns total.
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

// level_built[level] records the built rows (added to, when accumulate).
// Pairs a planning block can hold in LDS: the deepest planned level at
// maxDepth 12 has 2^11 nodes, i.e. at most 1024 sibling pairs.
constexpr uint32_t PLAN_MAX_PAIRS = 1024;

// Histogram items of num_pairs pairs (already in pairs[], written before a
// barrier): s_cnt / s_seg hold each pair's built node's rows and first entry
// (LDS, filled by the caller), s_first is LDS scratch of num_pairs words.
// Writes the chunk size, each pair's nchunks and item_first, and the items;
// every read-after-write inside the block goes through LDS.
__device__ void write_items(const Shape &sh, TreeCtl *ctl, int level, Pair *pairs,
                            HistItem *items, const uint32_t *s_cnt, const uint32_t *s_seg,
                            uint32_t *s_first, uint32_t num_pairs, uint32_t target_items,
                            uint32_t min_chunk, uint32_t *wave_tot, bool accumulate = false) {
    __shared__ uint32_t s_chunk;
    __shared__ uint32_t s_total;
    const int tid = threadIdx.x;
    // total built rows -> chunk size (accumulated in LDS)
    if (tid == 0) s_total = 0;
    __syncthreads();
    uint32_t part = 0;
    for (uint32_t k = tid; k < num_pairs; k += blockDim.x) part += s_cnt[k];
    part = wave_sum(part);
    if (lane_id() == 0) atomicAdd(&s_total, part);
    __syncthreads();
    if (tid == 0) {
        const uint64_t total = s_total;
        const uint32_t c = item_chunk(total, num_pairs, sh.hist_tiles, target_items, min_chunk);
        s_chunk = c;
        ctl->chunk = c;
        if (accumulate) ctl->level_built[level] += (uint32_t)total;
        else ctl->level_built[level] = (uint32_t)total;
    }
    __syncthreads();
    if (num_pairs <= 64 && tid < 64) {
        // Balance: the item chunk c above leaves room for one partial chunk per
        // (pair, tile), and the level's time is its largest item.  One
        // wavefront finds the smallest chunk c' whose per-pair chunk counts
        // still fit the same item budget (binary search between the lower
        // bound total / budget and c, which fits); each pair then splits its
        // rows into equal chunks of at most c'.
        // (32-bit arithmetic: 64-bit divisions in the loop cost microseconds)
        const uint32_t n = (uint32_t)tid < num_pairs ? s_cnt[tid] : 0u;
        const uint32_t K = (uint32_t)(item_budget(s_total, num_pairs, sh.hist_tiles,
                                                  target_items) / (uint64_t)sh.hist_tiles);
        uint32_t hi = s_chunk;
        uint32_t lo = s_total / K + (s_total % K != 0u);
        if (lo < min_chunk) lo = min_chunk;
        if (lo > hi) lo = hi;
        while (lo < hi) {                            // uniform across the wavefront
            const uint32_t mid = lo + (hi - lo) / 2;
            const uint32_t q = n / mid;
            if (wave_sum(q + (n - q * mid != 0u)) <= K) hi = mid; else lo = mid + 1;
        }
        if (tid == 0) s_chunk = lo;
    }
    __syncthreads();
    const uint32_t chunk = s_chunk;
    // the chunk of pair k: its rows in equal parts of at most `chunk`
    auto pair_chunk = [&](uint32_t cnt) {
        const uint32_t parts = (cnt + chunk - 1) / chunk;
        return parts ? (cnt + parts - 1) / parts : chunk;
    };
    // items per pair -> exclusive prefix
    for (uint32_t k = tid; k < num_pairs; k += blockDim.x) {
        const uint32_t pc = pair_chunk(s_cnt[k]);
        const uint32_t nch = (s_cnt[k] + pc - 1) / pc;
        pairs[k].nchunks = nch;
        s_first[k] = nch * (uint32_t)sh.hist_tiles;
    }
    __syncthreads();
    const uint32_t total_items = block_exclusive_scan(s_first, num_pairs, wave_tot);
    if (total_items > sh.item_cap) {
        // never write past the item list: the level gets no items and the
        // host reports the overflow after the tree
        for (uint32_t k = tid; k < num_pairs; k += blockDim.x) {
            pairs[k].item_first = 0;
            pairs[k].nchunks = 0;
        }
        if (tid == 0) {
            ctl->num_items = 0;
            ctl->overflow = 1;
        }
        return;
    }
    for (uint32_t k = tid; k < num_pairs; k += blockDim.x) pairs[k].item_first = s_first[k];
    if (tid == 0) ctl->num_items = total_items;
    for (uint32_t it = tid; it < total_items; it += blockDim.x) {
        // owning pair: last k with s_first[k] <= it
        uint32_t lo = 0, hi = num_pairs - 1;
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) >> 1;
            if (s_first[mid] <= it) lo = mid; else hi = mid - 1;
        }
        const uint32_t rel = it - s_first[lo];
        const uint32_t t = rel % (uint32_t)sh.hist_tiles, c = rel / (uint32_t)sh.hist_tiles;
        const uint32_t pc = pair_chunk(s_cnt[lo]);
        HistItem h;
        h.pair = lo;
        h.tile = t;
        h.start = s_seg[lo] + c * pc;
        h.count = min(pc, s_cnt[lo] - c * pc);
        items[it] = h;
    }
}

// The root's plan, by one workgroup of any size (a multiple of 64, at most
// 1024 threads).
__device__ void plan_root(const RootPlan &rp) {
    __shared__ uint32_t wave_tot[17];
    __shared__ uint32_t s_cnt[1], s_seg[1], s_first[1];
    if (threadIdx.x == 0) {
        uint32_t rows_active = rp.rows_active;
        if (rows_active == NONE) rows_active = rp.ctl->sampled;   // a sampled tree's kept rows
        rp.count[0] = rows_active;
        rp.seg_start[0] = 0;
        rp.ctl->level_active[0] = rows_active;
        rp.ctl->num_pairs = 1;
        rp.cover[0] = (float)rows_active;
        rp.bounds[0] = make_float2(rp.lo, rp.hi);
        Pair p = {};
        p.built = 0; p.derived = NONE; p.parent = NONE;
        rp.pairs[0] = p;
        s_cnt[0] = rows_active;
        s_seg[0] = 0;
    }
    __syncthreads();
    write_items(rp.sh, rp.ctl, 0, rp.pairs, rp.items, s_cnt, s_seg, s_first, 1, rp.target_items,
                rp.min_chunk, wave_tot);
}

__global__ __launch_bounds__(1024) void k_plan_root(RootPlan rp) { plan_root(rp); }

hipError_t launch_plan_root(hipStream_t s, const RootPlan &plan) {
    hipLaunchKernelGGL(k_plan_root, dim3(1), dim3(1024), 0, s, plan);
    return hipGetLastError();
}

// plan_level for at most 64 parents, by one wavefront (lane p: parent p,
// then pair p): the same outputs with no workgroup barrier.  Pair records are
// written whole by their own lane, after the chunking.
__device__ void plan_level_wave(const Shape &sh, const LevelArgs &la, uint32_t target_items,
                                uint32_t min_chunk, TreeCtl *ctl, const uint32_t *seg_start_prev,
                                uint32_t *seg_start_next, uint32_t *count,
                                const uint64_t *cursors, const TreeOut &out, Pair *pairs,
                                HistItem *items, const uint64_t *keys, float min_split_gain) {
    __shared__ uint32_t w_cnt[64], w_seg[64], w_first[64], w_parent[64];
    const uint32_t lane = (uint32_t)lane_id();
    const uint32_t num_prev = la.num_level >> 1;
    const uint32_t ls_prev = (la.level_start - 1) >> 1;
    const bool mine = lane < num_prev;
    bool split = false;
    uint32_t cl = 0, cr = 0, seg = 0;
    if (mine) {
        const uint32_t n = ls_prev + lane;
        const uint32_t cnt = count[n];
        const uint32_t left = (uint32_t)__hip_atomic_load(&cursors[(size_t)lane * CURSOR_STRIDE],
                                                          __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
        seg = seg_start_prev[lane];
        // parents decided in this pass carry keys (their model arrays are
        // written by other workgroups of it)
        split = keys ? key_splits(keys[(size_t)lane * KEY_STRIDE], cnt, min_split_gain)
                     : out.split[n].feature >= 0 && cnt >= 1;
        cl = split ? left : 0u;
        cr = split ? cnt - left : 0u;
        count[la.level_start + 2 * lane] = cl;
        count[la.level_start + 2 * lane + 1] = cr;
        out.cover[la.level_start + 2 * lane] = (float)cl;
        out.cover[la.level_start + 2 * lane + 1] = (float)cr;
        seg_start_next[2 * lane] = seg;
        seg_start_next[2 * lane + 1] = seg + cl;
    }
    const uint32_t act = wave_sum(cl + cr);
    if (lane == 0) ctl->level_active[la.level] = act;
    if (la.terminal) {
        if (lane == 0) { ctl->num_pairs = 0; ctl->num_items = 0; }
        return;
    }
    // sibling pairs for split parents, in parent order: the smaller child
    // builds, ties go left
    const uint64_t bal = __ballot(mine && split);
    const uint32_t num_pairs = (uint32_t)__popcll(bal);
    if (mine && split) {
        const uint32_t k = lanes_below(bal);
        const bool left_built = cl <= cr;
        w_cnt[k] = left_built ? cl : cr;
        w_seg[k] = left_built ? seg : seg + cl;
        w_parent[k] = lane | (left_built ? 0x80000000u : 0u);
    }
    if (lane == 0) ctl->num_pairs = num_pairs;
    if (num_pairs == 0) {
        if (lane == 0) ctl->num_items = 0;
        return;
    }
    wave_lds_sync();
    // lane k: pair k's built rows -> the level's chunk (write_items' rules)
    const bool own = lane < num_pairs;
    const uint32_t n = own ? w_cnt[lane] : 0u;
    const uint32_t total = wave_sum(n);
    const uint32_t c = item_chunk(total, num_pairs, sh.hist_tiles, target_items, min_chunk);
    if (lane == 0) {
        ctl->chunk = c;
        ctl->level_built[la.level] = total;
    }
    // the balance of write_items: the smallest chunk whose per-pair chunk
    // counts fit the item budget
    const uint32_t K = (uint32_t)(item_budget(total, num_pairs, sh.hist_tiles, target_items) /
                                  (uint64_t)sh.hist_tiles);
    uint32_t hi = c;
    uint32_t lo = total / K + (total % K != 0u);
    if (lo < min_chunk) lo = min_chunk;
    if (lo > hi) lo = hi;
    while (lo < hi) {                                // uniform across the wavefront
        const uint32_t mid = lo + (hi - lo) / 2;
        const uint32_t q = n / mid;
        if (wave_sum(q + (n - q * mid != 0u)) <= K) hi = mid; else lo = mid + 1;
    }
    const uint32_t chunk = lo;
    auto pair_chunk = [&](uint32_t cnt) {
        const uint32_t parts = (cnt + chunk - 1) / chunk;
        return parts ? (cnt + parts - 1) / parts : chunk;
    };
    const uint32_t pc = pair_chunk(n);
    const uint32_t nch = own ? (n + pc - 1) / pc : 0u;
    const uint32_t nit = nch * (uint32_t)sh.hist_tiles;
    const uint32_t inc = wave_inclusive_scan(nit);
    const uint32_t first = inc - nit;
    const uint32_t total_items = wave_last(inc);
    const bool fits = total_items <= sh.item_cap;
    if (own) {
        const uint32_t par = w_parent[lane];
        const uint32_t p = par & 0x7FFFFFFFu;
        const bool left_built = (par >> 31) != 0;
        Pair pr = {};
        pr.built = left_built ? 2 * p : 2 * p + 1;
        pr.derived = left_built ? 2 * p + 1 : 2 * p;
        pr.parent = p;
        // an overflowing level gets no items; the host reports it after the tree
        pr.item_first = fits ? first : 0u;
        pr.nchunks = fits ? nch : 0u;
        pairs[lane] = pr;
        w_first[lane] = first;
    }
    if (!fits) {
        if (lane == 0) { ctl->num_items = 0; ctl->overflow = 1; }
        return;
    }
    if (lane == 0) ctl->num_items = total_items;
    wave_lds_sync();
    for (uint32_t it = lane; it < total_items; it += 64) {
        // owning pair: the last k with w_first[k] <= it
        uint32_t a = 0, b = num_pairs - 1;
        while (a < b) {
            const uint32_t m = (a + b + 1) >> 1;
            if (w_first[m] <= it) a = m; else b = m - 1;
        }
        const uint32_t rel = it - w_first[a];
        const uint32_t t = rel % (uint32_t)sh.hist_tiles, ci = rel / (uint32_t)sh.hist_tiles;
        const uint32_t cnt = w_cnt[a];
        const uint32_t pca = pair_chunk(cnt);
        HistItem h;
        h.pair = a;
        h.tile = t;
        h.start = w_seg[a] + ci * pca;
        h.count = min(pca, cnt - ci * pca);
        items[it] = h;
    }
}

// Plan level d from level d-1's routed counts (decide_splits phase 2,
// Shaders.swift:1454-1488, with counts from the partition), run by one
// 1024-thread workgroup (at most 64 parents: by its first wavefront alone).  Thread p owns parent p (at most PLAN_MAX_PAIRS
// parents, so one pass); what later steps read back goes through LDS.  The
// partition cursors are read at device scope: the partition's last
// workgroup plans while the kernel that updated them is still resident.
__device__ void plan_level(const Shape &sh, const LevelArgs &la, uint32_t target_items,
                           uint32_t min_chunk, TreeCtl *ctl, const uint32_t *seg_start_prev,
                           uint32_t *seg_start_next, uint32_t *count, const uint64_t *cursors,
                           const TreeOut &out, Pair *pairs, HistItem *items,
                           const uint64_t *keys = nullptr, float min_split_gain = 0.0f) {
    __shared__ uint32_t wave_tot[17];
    __shared__ uint32_t s_active;
    __shared__ uint32_t s_idx[PLAN_MAX_PAIRS];       // split flag, then pair index
    __shared__ uint32_t s_cnt[PLAN_MAX_PAIRS], s_seg[PLAN_MAX_PAIRS], s_first[PLAN_MAX_PAIRS];
    const int tid = threadIdx.x;
    const uint32_t num_prev = la.num_level >> 1;
    const uint32_t ls_prev = (la.level_start - 1) >> 1;   // (2^d - 1 - 1) / 2 = 2^(d-1) - 1
    if (num_prev <= 64) {                            // uniform
        if (tid < 64)
            plan_level_wave(sh, la, target_items, min_chunk, ctl, seg_start_prev, seg_start_next,
                            count, cursors, out, pairs, items, keys, min_split_gain);
        return;
    }
    if (tid == 0) s_active = 0;
    // children of a split node share its interval: left [start, start+L),
    // right [start+L, start+count), with L from the partition's left cursor
    const uint32_t p = (uint32_t)tid;
    const bool mine = p < num_prev;
    bool split = false;
    uint32_t cl = 0, cr = 0, seg = 0;
    if (mine) {
        const uint32_t n = ls_prev + p;
        const uint32_t cnt = count[n];
        const uint32_t left = (uint32_t)__hip_atomic_load(&cursors[(size_t)p * CURSOR_STRIDE],
                                                          __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
        seg = seg_start_prev[p];
        split = keys ? key_splits(keys[(size_t)p * KEY_STRIDE], cnt, min_split_gain)
                     : out.split[n].feature >= 0 && cnt >= 1;
        cl = split ? left : 0u;
        cr = split ? cnt - left : 0u;
        count[la.level_start + 2 * p] = cl;
        count[la.level_start + 2 * p + 1] = cr;
        out.cover[la.level_start + 2 * p] = (float)cl;
        out.cover[la.level_start + 2 * p + 1] = (float)cr;
        seg_start_next[2 * p] = seg;
        seg_start_next[2 * p + 1] = seg + cl;
        s_idx[p] = split ? 1u : 0u;
    }
    const uint32_t act = wave_sum(cl + cr);
    __syncthreads();
    if (lane_id() == 0) atomicAdd(&s_active, act);
    __syncthreads();
    if (tid == 0) ctl->level_active[la.level] = s_active;
    if (la.terminal) {
        if (tid == 0) { ctl->num_pairs = 0; ctl->num_items = 0; }
        return;
    }
    // sibling pairs for split parents: the smaller child builds, ties go left
    const uint32_t num_pairs = block_exclusive_scan(s_idx, num_prev, wave_tot);
    if (mine && split) {
        const uint32_t k = s_idx[p];
        const bool left_built = cl <= cr;
        Pair pr = {};
        pr.built = left_built ? 2 * p : 2 * p + 1;
        pr.derived = left_built ? 2 * p + 1 : 2 * p;
        pr.parent = p;
        pairs[k] = pr;
        s_cnt[k] = left_built ? cl : cr;
        s_seg[k] = left_built ? seg : seg + cl;
    }
    if (tid == 0) ctl->num_pairs = num_pairs;
    __syncthreads();
    if (num_pairs == 0) {
        if (tid == 0) ctl->num_items = 0;
        return;
    }
    write_items(sh, ctl, la.level, pairs, items, s_cnt, s_seg, s_first, num_pairs, target_items,
                min_chunk, wave_tot);
}

__global__ __launch_bounds__(1024) void k_plan_level(
    Shape sh, LevelArgs la, uint32_t target_items, uint32_t min_chunk, TreeCtl *ctl,
    const uint32_t *seg_start_prev, uint32_t *seg_start_next, uint32_t *count,
    const uint64_t *cursors, const TreeOut out, Pair *pairs, HistItem *items) {
    plan_level(sh, la, target_items, min_chunk, ctl, seg_start_prev, seg_start_next, count,
               cursors, out, pairs, items);
}

hipError_t launch_plan_level(hipStream_t s, const Shape &sh, const LevelArgs &la,
                             uint32_t target_items, uint32_t min_chunk, TreeCtl *ctl,
                             const uint32_t *seg_start_prev, uint32_t *seg_start_next,
                             uint32_t *count, const uint64_t *cursors, const TreeOut out,
                             Pair *pairs, HistItem *items) {
    if ((la.num_level >> 1) > PLAN_MAX_PAIRS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_plan_level, dim3(1), dim3(1024), 0, s, sh, la, target_items, min_chunk,
                       ctl, seg_start_prev, seg_start_next, count, cursors, out, pairs, items);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// row partition (route_samples, Shaders.swift:1241-1311): one pass.  Every
// split node keeps its interval [start, start+count) of the order buffer; its
// children split that interval, left entries from the front and right
// entries from the back.  Each block covers PART_ENTRIES entries of one node, counts
// its lefts and rights, reserves both ranges with one atomic add each on the
// node's cursor (one packed 64-bit add: left count low, right count high; each
// node's cursor on its own 128-B line), and writes its entries there.  Entry order inside a child
// is not preserved; every consumer (histograms, counts, the next partition)
// is order-independent.  The left cursor ends as the node's left count.
// ---------------------------------------------------------------------------

// Large blocks keep the cursor atomics few (two per block); 8 entries per
// thread keep the kernel under 64 VGPRs, so two blocks share a CU.
constexpr int PART_THREADS = 1024;
constexpr int PART_PER_THREAD = PART_ENTRIES / PART_THREADS;
constexpr int PART_BLOCK = PART_THREADS * PART_PER_THREAD;
constexpr int PART_WAVES = PART_THREADS / 64;
constexpr int PART_SLICES = PART_PER_THREAD * PART_WAVES;
constexpr int PART_SLICES_PER_LANE = PART_SLICES / 64;
static_assert(PART_BLOCK == PART_ENTRIES, "partition block size");
static_assert(PART_SLICES % 64 == 0, "slice scan: whole slices per lane");

// One block's share of a node's partition: nvalid (<= PART_BLOCK) entries at
// src go to the node's interval dst[0, cnt), lefts from the front and rights
// from the back.  Both ranges are reserved with one packed 64-bit add on
// *cursor (left count low, right count high; both < 2^32, so the low word
// never carries).  s_mask is the split's category mask, in LDS.  With
// write_entries, returns (in every thread) whether this block's add was the
// one that reserved the node's last entries, and then the node's left count
// in *left_total.
__device__ __forceinline__ bool route_block(const NodeSplit sp, const uint32_t *s_mask, int32_t nb,
                                            const uint8_t *__restrict__ col,
                                            const Entry *__restrict__ src, uint32_t nvalid,
                                            uint32_t cnt, Entry *__restrict__ dst,
                                            uint64_t *cursor, bool write_entries,
                                            uint32_t *left_total = nullptr) {
    __shared__ uint32_t tot[PART_SLICES + 1];
    __shared__ uint64_t s_base;
    const int tid = threadIdx.x, w = tid >> 6;
    uint32_t x[PART_PER_THREAD], ex[PART_PER_THREAD];
    Entry e[PART_PER_THREAD];
#pragma unroll
    for (int k = 0; k < PART_PER_THREAD; ++k) {
        const uint32_t i = (uint32_t)(k * PART_THREADS + tid);
        x[k] = 0;
        e[k] = Entry{0u, 0u};
        if (i < nvalid) e[k] = load_entry_nt(src + i);
    }
#pragma unroll
    for (int k = 0; k < PART_PER_THREAD; ++k) {
        const uint32_t i = (uint32_t)(k * PART_THREADS + tid);
        if (i < nvalid) x[k] = bin_goes_left(col[e[k].row], sp, nb, s_mask) ? 1u : 0u;
    }
    // in-block exclusive prefix of the left flags in entry order (k, then lane)
#pragma unroll
    for (int k = 0; k < PART_PER_THREAD; ++k) {
        const uint32_t inc = wave_inclusive_scan(x[k]);
        ex[k] = inc - x[k];
        if (lane_id() == 63) tot[k * PART_WAVES + w] = inc;
    }
    __syncthreads();
    if (tid < 64) {
        // scan the PART_SLICES slice totals with one wave
        constexpr int SPL = PART_SLICES_PER_LANE;
        uint32_t v[SPL], s = 0;
#pragma unroll
        for (int j = 0; j < SPL; ++j) { v[j] = tot[tid * SPL + j]; s += v[j]; }
        const uint32_t inc = wave_inclusive_scan(s);
        uint32_t acc = inc - s;
#pragma unroll
        for (int j = 0; j < SPL; ++j) { tot[tid * SPL + j] = acc; acc += v[j]; }
        if (tid == 63) {
            const uint32_t nl = inc;
            tot[PART_SLICES] = nl;
            s_base = atomicAdd(reinterpret_cast<unsigned long long *>(cursor),
                               (unsigned long long)nl |
                                   ((unsigned long long)(nvalid - nl) << 32));
        }
    }
    if (!write_entries) return false;                // counts only (terminal level)
    __syncthreads();
    const uint32_t base_l = (uint32_t)s_base, base_r = (uint32_t)(s_base >> 32);
#pragma unroll
    for (int k = 0; k < PART_PER_THREAD; ++k) {
        const uint32_t i = (uint32_t)(k * PART_THREADS + tid);
        if (i >= nvalid) continue;
        const uint32_t le = ex[k] + tot[k * PART_WAVES + w];
        const uint32_t pos = x[k] ? base_l + le : cnt - 1u - (base_r + (i - le));
        store_entry_nt(dst + pos, e[k]);
    }
    if (base_l + base_r + nvalid != cnt) return false;
    if (left_total) *left_total = base_l + tot[PART_SLICES];
    return true;
}

// A persistent grid: each block computes the level's block prefix once and
// then takes logical blocks b, b + gridDim.x, ... (the logical blocks a level
// needs depend on its live rows, known only on the device; a sampled tree
// needs far fewer than the launch could hold).  The loop is software
// pipelined: while a block waits for its node cursor add (adds to one
// address serialize) and writes its entries, the next logical block's split
// record, mask and entries are already loading, so the bursts of loads and
// stores of consecutive logical blocks overlap.  Entry slot k of thread t is
// entry k * PART_THREADS + t of the logical block; a row's left flag lives
// as bit k of a per-thread mask, and its rank among the left rows of its
// wavefront slice comes from a ballot at store time.
template <bool IMPLICIT>
__global__ __launch_bounds__(PART_THREADS, 8) void k_route(
    Shape sh, LevelArgs la, const uint8_t *__restrict__ bins_fm, const Entry *__restrict__ order_in,
    Entry *__restrict__ order_out, const uint32_t *__restrict__ seg_start, uint32_t *count,
    const TreeOut out, uint64_t *cursors, int write_entries, RoutePlan rp, int has_plan,
    RouteDecide rd, int has_decide) {
    extern __shared__ uint32_t blk_prefix[];         // [num_level]: first block of each node
    __shared__ uint32_t s_mask[2][8];
    __shared__ uint32_t wave_tot[PART_WAVES + 1];
    __shared__ uint32_t tot[PART_SLICES + 1];
    __shared__ uint64_t s_base;
    const int tid = threadIdx.x, w = tid >> 6, lane = lane_id();
    // Logical block size: the level's live entries spread over whole rounds of
    // the grid (at most PART_BLOCK each, a multiple of 64), so every workgroup
    // takes about the same number of entries instead of a last round of
    // 8,192-entry blocks on part of the grid.  Each split node adds at most one
    // partial block, which the rounds reserve.
    __shared__ uint32_t s_live, s_nsplit, s_bsz;
    if (tid == 0) { s_live = 0; s_nsplit = 0; }
    __syncthreads();
    {
        uint32_t live = 0, nsplit = 0;
        for (uint32_t l = threadIdx.x; l < la.num_level; l += PART_THREADS) {
            const uint32_t nn = la.level_start + l;
            const bool split = has_decide ? key_splits(rd.keys[(size_t)l * KEY_STRIDE], count[nn],
                                                       rd.sp.min_split_gain)
                                          : out.split[nn].feature >= 0 && count[nn] >= 1;
            blk_prefix[l] = split ? count[nn] : 0u;
            live += blk_prefix[l];
            nsplit += split ? 1u : 0u;
        }
        live = wave_sum(live);
        nsplit = wave_sum(nsplit);
        if (lane == 0 && (live | nsplit)) {
            atomicAdd(&s_live, live);
            atomicAdd(&s_nsplit, nsplit);
        }
    }
    __syncthreads();
    if (tid == 0) {
        const uint64_t live = s_live, nsplit = s_nsplit, g = gridDim.x;
        const uint64_t rounds = ((live + PART_BLOCK - 1) / PART_BLOCK + nsplit + g - 1) / g;
        const uint64_t slots = rounds * g > nsplit ? rounds * g - nsplit : 1;
        uint64_t bsz = (live + slots - 1) / slots;
        bsz = (bsz + 63) / 64 * 64;
        s_bsz = (uint32_t)(bsz < 64 ? 64 : bsz > PART_BLOCK ? PART_BLOCK : bsz);
    }
    __syncthreads();
    const uint32_t bsz = s_bsz;
    // blocks per split node of the routed level, and their prefix
    for (uint32_t l = threadIdx.x; l < la.num_level; l += PART_THREADS)
        blk_prefix[l] = (blk_prefix[l] + bsz - 1) / bsz;
    __syncthreads();
    const uint32_t total_blocks = block_exclusive_scan(blk_prefix, la.num_level, wave_tot);
    const uint64_t *keys = has_decide ? rd.keys : nullptr;
    // decide mode: node l's model arrays, children's sums and bounds, by
    // workgroup l % gridDim.x before its blocks (nothing in this pass reads
    // them: routing and the planner take the splits from the keys; made at
    // the end instead, they lengthened the pass's tail: 10M x 100 fit +0.3 ms)
    auto decide_mine = [&]() {
        if (!has_decide || tid != 0) return;
        for (uint32_t l = blockIdx.x; l < la.num_level; l += gridDim.x) {
            const uint32_t n = la.level_start + l;
            if (count[n] < 1) {
                out.split[n] = NodeSplit{-1, 0, 0};
                out.leaf[n] = 0.0f;
                out.gain[n] = 0.0f;
                continue;
            }
            const uint64_t k = rd.keys[(size_t)l * KEY_STRIDE];
            const float bg = k ? key_float((uint32_t)(k >> 32)) : -INFINITY;
            decide_apply(rd.sp, rd.cols, n, l, key_feature(k), bg, rd.results, rd.node_g[n],
                         rd.node_h[n], rd.bounds[n], rd.ctl->max_gh[0], rd.ctl->max_gh[1],
                         rd.node_g, rd.node_h, rd.bounds, rd.monotone, out);
        }
    };
    decide_mine();
    uint32_t b = blockIdx.x;
    if (b >= total_blocks) {                         // uniform per block
        // nothing to partition: the first workgroup plans alone
        if (has_plan && total_blocks == 0 && blockIdx.x == 0)
            plan_level(sh, rp.next, rp.target_items, rp.min_chunk, rp.ctl, seg_start, rp.seg_next,
                       count, cursors, out, rp.pairs, rp.items, keys, rd.sp.min_split_gain);
        return;
    }

    // logical block b: its node slot, segment, count, first entry, split and
    // the sides whose entries are written (bit 0 left, bit 1 right)
    struct Blk {
        uint32_t l, start, cnt, first, nvalid, sides;
        NodeSplit sp;
    };
    auto locate = [&](uint32_t bb, Blk &k) {
        // owning node: the largest l with blk_prefix[l] <= bb (it has blocks)
        uint32_t lo = 0, hi = la.num_level - 1;
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) >> 1;
            if (blk_prefix[mid] <= bb) lo = mid; else hi = mid - 1;
        }
        const uint32_t n = la.level_start + lo;
        k.l = lo;
        k.start = seg_start[lo];
        k.cnt = count[n];
        k.first = (bb - blk_prefix[lo]) * bsz;
        k.nvalid = min(bsz, k.cnt - k.first);
        k.sides = 3u;
        if (has_decide) {
            const int f = key_feature(rd.keys[(size_t)lo * KEY_STRIDE]);
            const SplitResult *r = rd.results + (size_t)lo * rd.cols + f;
            k.sp = NodeSplit{f, r->bin, r->flags};
            if (write_entries == 2)                  // the plan's built child only
                k.sides = r->hl_int <= rd.node_h[n] - r->hl_int ? 1u : 2u;
        } else {
            k.sp = out.split[n];
        }
    };
    // word w of the node's category mask (decide_node's: the winning
    // feature's subset for a categorical split, else zeros)
    auto mask_word = [&](const Blk &k, int wd) -> uint32_t {
        if (!has_decide) return out.mask[(size_t)(la.level_start + k.l) * 8 + wd];
        if (!(k.sp.flags & FLAG_CATEGORICAL)) return 0u;
        return rd.results[(size_t)k.l * rd.cols + k.sp.feature].mask[wd];
    };
    auto load_entries = [&](const Blk &k, Entry (&e)[PART_PER_THREAD]) {
        const uint32_t e0 = k.start + k.first;
        const Entry *src = order_in + e0;
        // implicit input: entry j is row j with its packed word
        const uint32_t *src_q = reinterpret_cast<const uint32_t *>(order_in) + e0;
#pragma unroll
        for (int j = 0; j < PART_PER_THREAD; ++j) {
            const uint32_t i = (uint32_t)(j * PART_THREADS + tid);
            e[j] = Entry{0u, 0u};
            if (i < k.nvalid) {
                if constexpr (IMPLICIT) e[j] = Entry{e0 + i, __builtin_nontemporal_load(src_q + i)};
                else e[j] = load_entry_nt(src + i);
            }
        }
    };

    Blk cur;
    Entry e[PART_PER_THREAD];
    locate(b, cur);
    if (tid < 8) s_mask[0][tid] = mask_word(cur, tid);
    load_entries(cur, e);
    int buf = 0;
    __syncthreads();
    for (;;) {
        const uint32_t bn = b + gridDim.x;
        const bool has_next = bn < total_blocks;     // uniform per block
        // left flags of this block's entries
        const uint8_t *col = bins_fm + (size_t)cur.sp.feature * (size_t)sh.rows;
        uint32_t bins[PART_PER_THREAD];
#pragma unroll
        for (int j = 0; j < PART_PER_THREAD; ++j) {
            const uint32_t i = (uint32_t)(j * PART_THREADS + tid);
            bins[j] = i < cur.nvalid ? col[e[j].row] : 0u;
        }
        uint32_t left = 0;
#pragma unroll
        for (int j = 0; j < PART_PER_THREAD; ++j) {
            const uint32_t i = (uint32_t)(j * PART_THREADS + tid);
            if (i < cur.nvalid && bin_goes_left(bins[j], cur.sp, sh.num_bins, s_mask[buf]))
                left |= 1u << j;
        }
        // left rows per wavefront slice (slice = (entry slot j, wavefront))
#pragma unroll
        for (int j = 0; j < PART_PER_THREAD; ++j) {
            const uint64_t bal = __ballot((left >> j) & 1u);
            if (lane == 0) tot[j * PART_WAVES + w] = (uint32_t)__popcll(bal);
        }
        __syncthreads();
        uint64_t old = 0;
        if (tid < 64) {
            // scan the PART_SLICES slice totals with one wave
            constexpr int SPL = PART_SLICES_PER_LANE;
            uint32_t v[SPL], sum = 0;
#pragma unroll
            for (int j = 0; j < SPL; ++j) { v[j] = tot[tid * SPL + j]; sum += v[j]; }
            const uint32_t inc = wave_inclusive_scan(sum);
            uint32_t acc = inc - sum;
#pragma unroll
            for (int j = 0; j < SPL; ++j) { tot[tid * SPL + j] = acc; acc += v[j]; }
            if (tid == 63)
                old = atomicAdd(reinterpret_cast<unsigned long long *>(
                                    &cursors[(size_t)cur.l * CURSOR_STRIDE]),
                                (unsigned long long)inc |
                                    ((unsigned long long)(cur.nvalid - inc) << 32));
        }
        // the next logical block loads while the cursor add is in flight
        Blk nxt = cur;
        Entry en[PART_PER_THREAD];
        if (has_next) {
            locate(bn, nxt);
            if (tid < 8) s_mask[buf ^ 1][tid] = mask_word(nxt, tid);
            load_entries(nxt, en);
        }
        if (tid == 63) s_base = old;
        __syncthreads();
        if (write_entries) {
            const uint32_t base_l = (uint32_t)s_base, base_r = (uint32_t)(s_base >> 32);
            Entry *dst = order_out + cur.start;
#pragma unroll
            for (int j = 0; j < PART_PER_THREAD; ++j) {
                const uint32_t i = (uint32_t)(j * PART_THREADS + tid);
                const bool is_left = (left >> j) & 1u;
                const uint32_t le =
                    tot[j * PART_WAVES + w] + lanes_below(__ballot(is_left));
                if (i >= cur.nvalid || !(cur.sides & (is_left ? 1u : 2u))) continue;
                const uint32_t pos = is_left ? base_l + le : cur.cnt - 1u - (base_r + (i - le));
                store_entry_nt(dst + pos, e[j]);
            }
        }
        __syncthreads();                             // tot / s_base reuse, the next mask
        if (!has_next) break;
        cur = nxt;
#pragma unroll
        for (int j = 0; j < PART_PER_THREAD; ++j) e[j] = en[j];
        buf ^= 1;
        b = bn;
    }
    if (has_plan) {
        // the last of the busy workgroups plans the next level.  Every cursor
        // add of a workgroup has returned before its count add, and the
        // planner reads the cursors at device scope.
        __shared__ uint32_t s_last;
        const uint32_t busy = min(gridDim.x, total_blocks);
        if (tid == 0) s_last = atomicAdd(rp.done, 1u) == busy - 1u ? 1u : 0u;
        __syncthreads();
        if (s_last) {
            if (tid == 0) atomicExch(rp.done, 0u);
            plan_level(sh, rp.next, rp.target_items, rp.min_chunk, rp.ctl, seg_start, rp.seg_next,
                       count, cursors, out, rp.pairs, rp.items, keys, rd.sp.min_split_gain);
        }
    }
}

hipError_t launch_route(hipStream_t s, const Shape &sh, const LevelArgs &la,
                        const uint8_t *bins_fm, const Entry *order_in, Entry *order_out,
                        const uint32_t *seg_start, uint32_t *count, const TreeOut out,
                        uint64_t *cursors, uint32_t max_blocks, bool write_entries,
                        const RoutePlan *plan, bool implicit_in, const RouteDecide *decide,
                        bool built_only) {
    // cursors were zeroed by this level's k_decide (or, with decide, by
    // launch_split's reduction)
    if (max_blocks < 1) return hipErrorInvalidValue;
    if (decide && (!decide->keys || !decide->results || !decide->ctl || decide->cols < 1))
        return hipErrorInvalidValue;
    if (built_only && (!decide || !write_entries)) return hipErrorInvalidValue;
    RoutePlan rp{};
    if (plan) {
        if ((plan->next.num_level >> 1) > PLAN_MAX_PAIRS || !plan->done) return hipErrorInvalidValue;
        rp = *plan;
    }
    const size_t lds = (size_t)la.num_level * sizeof(uint32_t);
    auto *kern = implicit_in ? &k_route<true> : &k_route<false>;
    hipLaunchKernelGGL(kern, dim3(max_blocks), dim3(PART_THREADS), lds, s, sh, la, bins_fm,
                       order_in, order_out, seg_start, count, out, cursors,
                       write_entries ? (built_only ? 2 : 1) : 0, rp, plan ? 1 : 0,
                       decide ? *decide : RouteDecide{},
                       decide ? 1 : 0);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Boruta shadow columns (shadow_perm + shadow_bins, Shaders.swift:1596-1631):
// fm2 [2F][rows] = the real bins, then each column's bins row-permuted by a
// 4-round Feistel network over 2*hb bits with cycle walking (a bijection of
// [0, rows), so the walk ends for every row).
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t shadow_perm(uint32_t i, uint32_t n, uint32_t hb,
                                                uint32_t seed) {
    const uint32_t mask = (1u << hb) - 1u;
    do {
        uint32_t L = i >> hb, R = i & mask;
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) {
            const uint32_t t = R;
            R = L ^ (wang_hash(R ^ (seed + r * 0x9E3779B9u)) & mask);
            L = t;
        }
        i = (L << hb) | R;
    } while (i >= n);
    return i;
}

__global__ __launch_bounds__(256) void k_shadow_bins(const uint8_t *__restrict__ fm, int64_t rows,
                                                     int32_t cols, uint32_t hb, uint32_t seed,
                                                     uint8_t *__restrict__ fm2) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int32_t f = blockIdx.y;
    if (i >= rows) return;
    fm2[(int64_t)f * rows + i] = fm[(int64_t)f * rows + i];
    const uint32_t j = shadow_perm((uint32_t)i, (uint32_t)rows, hb, seed ^ wang_hash((uint32_t)f + 1u));
    fm2[(int64_t)(cols + f) * rows + i] = fm[(int64_t)f * rows + j];
}

hipError_t launch_shadow_bins(hipStream_t s, const uint8_t *fm, int64_t rows, int32_t cols,
                              uint32_t half_bits, uint32_t seed, uint8_t *fm2) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (rows > 0xFFFFFFFFLL || 2 * half_bits > 32 || ((uint64_t)1 << (2 * half_bits)) < (uint64_t)rows)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_shadow_bins, dim3((unsigned)((rows + 255) / 256), (unsigned)cols),
                       dim3(256), 0, s, fm, rows, cols, half_bits, seed, fm2);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Leaf renewal for the L1 and quantile objectives (Booster.swift:634-639,
// :1253-1290, :1596-1615): the residuals y - preds of every step-th row,
// grouped by the leaf the row reaches; a leaf with >= 4 of them becomes
// lr * min(max(r_(k), lo), hi), r_(k) the k-th smallest with
// k = min(n-1, (int)((float)n * q)).  Grouping is a counting sort by leaf
// (per-block LDS counts, one global add per non-empty leaf and block); the
// order statistic is an MSB-first radix select over order-preserving keys,
// one workgroup per leaf.
// ---------------------------------------------------------------------------

constexpr int RENEW_THREADS = 1024;

__device__ __forceinline__ uint32_t walk_binned_row(const uint8_t *__restrict__ bins_fm,
                                                    int64_t rows, int32_t nb, int32_t max_depth,
                                                    const TreeOut &tree, int64_t i) {
    uint32_t n = 0;
    for (int32_t d = 0; d < max_depth; ++d) {
        const NodeSplit s = tree.split[n];
        if (s.feature < 0) break;
        const uint32_t b = bins_fm[(int64_t)s.feature * rows + i];
        n = 2 * n + 1 + (bin_goes_left(b, s, nb, tree.mask + (size_t)n * 8) ? 0u : 1u);
    }
    return n;
}

// Leaf and residual key of each sampled row; per-leaf counts (cnt pre-zeroed).
__global__ __launch_bounds__(RENEW_THREADS) void k_renew_collect(
    const uint8_t *__restrict__ bins_fm, int64_t rows, int32_t nb, int32_t max_depth,
    TreeOut tree, const float *__restrict__ labels, const float *__restrict__ preds,
    int64_t step, uint32_t ns, uint32_t total_nodes, uint32_t *__restrict__ leaf_of,
    uint32_t *__restrict__ keys, uint32_t *__restrict__ cnt) {
    extern __shared__ uint32_t rc_lds[];             // [total_nodes]
    for (uint32_t k = threadIdx.x; k < total_nodes; k += RENEW_THREADS) rc_lds[k] = 0;
    __syncthreads();
    const uint32_t s = blockIdx.x * RENEW_THREADS + threadIdx.x;
    if (s < ns) {
        const int64_t i = (int64_t)s * step;
        const uint32_t n = walk_binned_row(bins_fm, rows, nb, max_depth, tree, i);
        leaf_of[s] = n;
        keys[s] = float_key(labels[i] - preds[i]);
        atomicAdd(&rc_lds[n], 1u);
    }
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < total_nodes; k += RENEW_THREADS)
        if (rc_lds[k]) atomicAdd(&cnt[k], rc_lds[k]);
}

// Exclusive prefix of the per-leaf counts: segment starts and cursors.
__global__ __launch_bounds__(1024) void k_renew_offsets(const uint32_t *__restrict__ cnt,
                                                        uint32_t total_nodes, uint32_t *off,
                                                        uint32_t *cursor) {
    __shared__ uint32_t wave_tot[17];
    for (uint32_t k = threadIdx.x; k < total_nodes; k += blockDim.x) off[k] = cnt[k];
    __syncthreads();
    block_exclusive_scan(off, total_nodes, wave_tot);
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < total_nodes; k += blockDim.x) cursor[k] = off[k];
}

// Keys into their leaf's segment (order inside a segment is free).
__global__ __launch_bounds__(RENEW_THREADS) void k_renew_scatter(
    const uint32_t *__restrict__ leaf_of, const uint32_t *__restrict__ keys, uint32_t ns,
    uint32_t total_nodes, uint32_t *cursor, uint32_t *__restrict__ seg) {
    extern __shared__ uint32_t rs_lds[];             // [2 * total_nodes]: counts, bases
    uint32_t *s_cnt = rs_lds, *s_base = rs_lds + total_nodes;
    for (uint32_t k = threadIdx.x; k < total_nodes; k += RENEW_THREADS) s_cnt[k] = 0;
    __syncthreads();
    const uint32_t s = blockIdx.x * RENEW_THREADS + threadIdx.x;
    uint32_t n = 0, local = 0;
    if (s < ns) {
        n = leaf_of[s];
        local = atomicAdd(&s_cnt[n], 1u);
    }
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < total_nodes; k += RENEW_THREADS)
        if (s_cnt[k]) s_base[k] = atomicAdd(&cursor[k], s_cnt[k]);
    __syncthreads();
    if (s < ns) seg[s_base[n] + local] = keys[s];
}

// One workgroup per node: radix select of the k-th key (4 passes of 8 bits),
// then the renewed leaf.  With delta != null (leaf-wise) a changed leaf
// records delta = new - old; every other node gets delta = 0.
__global__ __launch_bounds__(256) void k_renew_select(const uint32_t *__restrict__ seg,
                                                      const uint32_t *__restrict__ off,
                                                      const uint32_t *__restrict__ cnt, float q,
                                                      float lr, const float2 *__restrict__ bounds,
                                                      TreeOut tree, float *delta) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_prefix, s_k;
    const uint32_t n = blockIdx.x;
    const uint32_t c = cnt[n];
    if (c < 4) {
        if (delta && threadIdx.x == 0) delta[n] = 0.0f;
        return;
    }
    const uint32_t *sg = seg + off[n];
    if (threadIdx.x == 0) {
        uint32_t k = (uint32_t)((float)c * q);
        s_k = k < c - 1 ? k : c - 1;
        s_prefix = 0;
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[threadIdx.x] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix;
        const uint32_t hi_mask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
        for (uint32_t j = threadIdx.x; j < c; j += 256) {
            const uint32_t key = sg[j];
            if ((key & hi_mask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFFu], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t k = s_k, cum = 0, b = 0;
            for (; b < 255; ++b) {
                if (cum + hist[b] > k) break;
                cum += hist[b];
            }
            s_prefix = prefix | (b << shift);
            s_k = k - cum;
        }
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    const float2 bd = bounds[n];
    float v = key_float(s_prefix);
    v = v > bd.x ? v : bd.x;                         // min(max(q, lo), hi)
    v = v < bd.y ? v : bd.y;
    v = lr * v;
    if (delta) {
        const float old = tree.leaf[n];
        delta[n] = v != old ? v - old : 0.0f;
        tree.leaf[n] = v;
    } else {
        tree.leaf[n] = v;
    }
}

size_t renew_sample_count(int64_t rows) {
    int64_t step = rows / 262144;
    if (step < 1) step = 1;
    return (size_t)((rows + step - 1) / step);
}

hipError_t launch_renew(hipStream_t s, const uint8_t *bins_fm, int64_t rows, int32_t nb,
                        int32_t max_depth, TreeOut tree, const float *labels,
                        const float *preds, const float2 *bounds, float q, float lr,
                        uint32_t *leaf_of, uint32_t *keys, uint32_t *seg, uint32_t *cnt,
                        uint32_t *off, uint32_t *cursor, float *delta) {
    int64_t step = rows / 262144;
    if (step < 1) step = 1;
    const uint32_t ns = (uint32_t)renew_sample_count(rows);
    const uint32_t total = (1u << (max_depth + 1)) - 1u;
    const unsigned blocks = (ns + RENEW_THREADS - 1) / RENEW_THREADS;
    hipError_t e = hipMemsetAsync(cnt, 0, (size_t)total * sizeof(uint32_t), s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_renew_collect, dim3(blocks), dim3(RENEW_THREADS),
                       (size_t)total * sizeof(uint32_t), s, bins_fm, rows, nb, max_depth, tree,
                       labels, preds, step, ns, total, leaf_of, keys, cnt);
    hipLaunchKernelGGL(k_renew_offsets, dim3(1), dim3(1024), 0, s, cnt, total, off, cursor);
    hipLaunchKernelGGL(k_renew_scatter, dim3(blocks), dim3(RENEW_THREADS),
                       (size_t)total * 2 * sizeof(uint32_t), s, leaf_of, keys, ns, total, cursor,
                       seg);
    hipLaunchKernelGGL(k_renew_select, dim3(total), dim3(256), 0, s, seg, off, cnt, q, lr,
                       bounds, tree, delta);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// leaf-wise (best-first) growth: leaf_init (:683-716), leaf_pick_apply
// (:720-871), leaf_step (:879-1091) and the segment partition
// (partition_count/scan/scatter, :520-620, here one pass like the level-wise
// one: entry order inside a child is not kept, and nothing depends on it).
// Every step is a fixed chain of launches (pick with the previous step's
// evaluations, route, plan, histograms, reduce, split) that read the device
// state; once the tree is finished the chain early-outs, so the host never
// waits inside a tree.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float lw_leaf_value(const SplitParams &sp, int64_t g, int64_t h,
                                               float g_inv, float h_inv, float lo, float hi) {
    const float G = (float)g * g_inv, H = (float)h * h_inv;
    return sp.learning_rate * clampf(-G / (H + sp.lambda), lo, hi);
}

__global__ __launch_bounds__(1024) void k_lw_init(Shape sh, LWArgs a, TreeCtl *ctl, LWState *st,
                                                  LWOpen *open, uint32_t *slot_seg,
                                                  uint32_t *slot_count, Pair *pairs,
                                                  HistItem *items, TreeOut out, int sampled) {
    __shared__ uint32_t wave_tot[17];
    __shared__ uint32_t s_cnt[1], s_seg[1], s_first[1];
    const int tid = threadIdx.x;
    for (int n = tid; n < a.total_nodes; n += blockDim.x) {
        const NodeSplit leaf = {-1, 0, 0};
        out.split[n] = leaf;
        out.leaf[n] = 0.0f;
        out.gain[n] = 0.0f;
        out.cover[n] = 0.0f;
    }
    for (int k = tid; k < a.total_nodes * 8; k += blockDim.x) out.mask[k] = 0u;
    const uint32_t n0 = sampled ? ctl->sampled : a.rows;   // the tree's rows
    if (tid == 0) {
        LWState s = {};
        s.leaves = 1;
        s.open_count = 1;
        s.next_slot = 1;
        s.eval_first = 0;
        s.eval_count = 1;
        *st = s;
        LWOpen o = {};
        o.node = 0;
        o.seg = 0;
        o.count = n0;
        o.depth = 0;
        o.slot = 0;
        o.best_f = -1;
        o.lo = -INFINITY;
        o.hi = INFINITY;
        o.best.gain = -INFINITY;
        open[0] = o;
        slot_seg[0] = 0;
        slot_count[0] = n0;
        Pair p = {};
        p.built = 0; p.derived = NONE; p.parent = NONE;
        pairs[0] = p;
        ctl->num_pairs = 1;
        ctl->level_active[0] = n0;
        out.cover[0] = (float)n0;
        s_cnt[0] = n0;
        s_seg[0] = 0;
    }
    __syncthreads();
    write_items(sh, ctl, 0, pairs, items, s_cnt, s_seg, s_first, 1, a.target_items, a.min_chunk,
                wave_tot, true);
}

hipError_t launch_lw_init(hipStream_t s, const Shape &sh, const LWArgs &a, TreeCtl *ctl,
                          LWState *st, LWOpen *open, uint32_t *slot_seg, uint32_t *slot_count,
                          Pair *pairs, HistItem *items, const TreeOut out, bool sampled) {
    hipLaunchKernelGGL(k_lw_init, dim3(1), dim3(1024), 0, s, sh, a, ctl, st, open, slot_seg,
                       slot_count, pairs, items, out, sampled ? 1 : 0);
    return hipGetLastError();
}

// Best split of newly evaluated leaf eval_first + w: argmax over features
// (strict '>', lowest feature wins), one wavefront per leaf.
__device__ void lw_eval_leaf(int w, const Shape &sh, const SplitParams &sp, const LWState *st,
                             LWOpen *open, const SplitResult *__restrict__ results,
                             const int64_t *slot_g, const int64_t *slot_h, const TreeCtl *ctl,
                             const TreeOut &out) {
    const int lane = lane_id();
    if ((uint32_t)w >= st->eval_count) return;
    const uint32_t e = st->eval_first + (uint32_t)w;
    const int32_t slot = open[e].slot;
    if (slot < 0) return;
    const int F = sh.cols;
    float bg = -INFINITY;
    int bf = 0x7FFFFFFF;
    for (int f = lane; f < F; f += 64) {
        const float g = results[(size_t)slot * F + f].gain;
        if (g > bg) { bg = g; bf = f; }
    }
    wave_argmax(bg, bf);
    if (lane != 0) return;
    LWOpen o = open[e];
    o.g = slot_g[slot];
    o.h = slot_h[slot];
    if (bf != 0x7FFFFFFF) {
        o.best = results[(size_t)slot * F + bf];
        o.best_f = bf;
    } else {
        o.best_f = -1;
        o.best.gain = -INFINITY;
    }
    open[e] = o;
    if (o.node == 0) {                               // the root's own leaf value
        const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
        const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;
        out.leaf[0] = lw_leaf_value(sp, o.g, o.h, g_inv, h_inv, o.lo, o.hi);
    }
}

// The last step's evaluations (the root's, when the tree never splits).
__global__ __launch_bounds__(128) void k_lw_eval(Shape sh, SplitParams sp, const LWState *st,
                                                 LWOpen *open,
                                                 const SplitResult *__restrict__ results,
                                                 const int64_t *slot_g, const int64_t *slot_h,
                                                 const TreeCtl *ctl, TreeOut out) {
    if (st->done) return;
    lw_eval_leaf(threadIdx.x >> 6, sh, sp, st, open, results, slot_g, slot_h, ctl, out);
}

hipError_t launch_lw_eval(hipStream_t s, const Shape &sh, const SplitParams &sp,
                          const LWState *st, LWOpen *open, const SplitResult *results,
                          const int64_t *slot_g, const int64_t *slot_h, const TreeCtl *ctl,
                          const TreeOut out) {
    hipLaunchKernelGGL(k_lw_eval, dim3(1), dim3(128), 0, s, sh, sp, st, open, results, slot_g,
                       slot_h, ctl, out);
    return hipGetLastError();
}

// Evaluate the leaves the previous step built, then pick the open leaf with
// the largest gain > minSplitGain (lowest index wins), write its split, its
// children's statistics, bounds and leaf values, and set up the partition of
// its segment (the partition cursor starts at zero).
__global__ __launch_bounds__(128) void k_lw_pick(Shape sh, SplitParams sp, LWArgs a, LWState *st,
                                                 LWOpen *open,
                                                 const SplitResult *__restrict__ results,
                                                 const int64_t *slot_g, const int64_t *slot_h,
                                                 const int8_t *monotone, TreeCtl *ctl,
                                                 uint64_t *cursor, TreeOut out) {
    const int lane = lane_id(), wv = threadIdx.x >> 6;
    if (st->done) {
        if (threadIdx.x == 0) {
            ctl->num_items = 0;
            ctl->num_pairs = 0;
        }
        return;
    }
    lw_eval_leaf(wv, sh, sp, st, open, results, slot_g, slot_h, ctl, out);
    __syncthreads();
    if (wv != 0) return;
    if (lane == 0) {
        ctl->num_items = 0;                          // nothing to build unless planned
        ctl->num_pairs = 0;
    }
    if ((int32_t)st->leaves >= a.num_leaves) {
        if (lane == 0) st->done = 1;
        return;
    }
    const uint32_t n_open = st->open_count;
    float bg = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (uint32_t i = (uint32_t)lane; i < n_open; i += 64) {
        const LWOpen &o = open[i];
        const float g = o.best.gain;
        if (o.best_f >= 0 && isfinite(g) && g > sp.min_split_gain && g > bg) {
            bg = g;
            bi = (int)i;
        }
    }
    wave_argmax(bg, bi);
    if (lane != 0) return;
    if (bi == 0x7FFFFFFF) {
        st->done = 1;
        return;
    }
    const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
    const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;
    const LWOpen o = open[bi];
    const SplitResult r = o.best;
    const int32_t n = o.node, bf = o.best_f;
    const bool cat = (r.flags & FLAG_CATEGORICAL) != 0;
    const NodeSplit ns = {bf, r.bin, r.flags};
    out.split[n] = ns;
    out.leaf[n] = 0.0f;
    out.gain[n] = r.gain;
    for (int w = 0; w < 8; ++w) out.mask[(size_t)n * 8 + w] = cat ? r.mask[w] : 0u;
    // children (monotone bounds: Shaders.swift:1424-1443)
    const int64_t lg = r.gl_int, lh = r.hl_int, rg = o.g - r.gl_int, rh = o.h - r.hl_int;
    float llo = o.lo, lhi = o.hi, rlo = o.lo, rhi = o.hi;
    const int cst = cat ? 0 : (int)monotone[bf];
    if (cst != 0) {
        const float vl = -r.gl / (r.hl + sp.lambda);
        const float gr = (float)rg * g_inv, hr = (float)rh * h_inv;
        const float vr = -gr / (hr + sp.lambda);
        const float mid = clampf(0.5f * (vl + vr), o.lo, o.hi);
        if (cst > 0) { lhi = fminf(lhi, mid); rlo = fmaxf(rlo, mid); }
        else { llo = fmaxf(llo, mid); rhi = fminf(rhi, mid); }
    }
    const int32_t lc = 2 * n + 1, rc = 2 * n + 2;
    out.leaf[lc] = lw_leaf_value(sp, lg, lh, g_inv, h_inv, llo, lhi);
    out.leaf[rc] = lw_leaf_value(sp, rg, rh, g_inv, h_inv, rlo, rhi);
    const uint32_t i0 = n_open;
    LWOpen c = {};
    c.depth = o.depth + 1;
    c.slot = -1;
    c.best_f = -1;
    c.best.gain = -INFINITY;
    c.node = lc; c.g = lg; c.h = lh; c.lo = llo; c.hi = lhi;
    open[i0] = c;
    c.node = rc; c.g = rg; c.h = rh; c.lo = rlo; c.hi = rhi;
    open[i0 + 1] = c;
    open[bi].best_f = -1;
    open[bi].best.gain = -INFINITY;
    st->pick = (uint32_t)bi;
    st->pick_node = n;
    st->pick_depth = o.depth;
    st->pick_slot = o.slot;
    st->child0 = i0;
    st->open_count = n_open + 2;
    st->eval_count = 0;
    st->src = o.seg;
    st->dst = o.seg < a.rows ? o.seg + a.rows : o.seg - a.rows;
    st->count = o.count;
    *cursor = 0ull;
    st->feature = bf;
    st->bin = r.bin;
    st->flags = r.flags;
    for (int w = 0; w < 8; ++w) st->mask[w] = cat ? r.mask[w] : 0u;
}

hipError_t launch_lw_pick(hipStream_t s, const Shape &sh, const SplitParams &sp, const LWArgs &a,
                          LWState *st, LWOpen *open, const SplitResult *results,
                          const int64_t *slot_g, const int64_t *slot_h, const int8_t *monotone,
                          TreeCtl *ctl, uint64_t *cursor, const TreeOut out) {
    hipLaunchKernelGGL(k_lw_pick, dim3(1), dim3(128), 0, s, sh, sp, a, st, open, results, slot_g,
                       slot_h, monotone, ctl, cursor, out);
    return hipGetLastError();
}

// Every open-list node's leaf bounds into bounds[node] (leaf renewal reads
// them for the finished tree's leaves).
__global__ void k_lw_bounds(const LWState *st, const LWOpen *open, float2 *bounds) {
    const uint32_t n = st->open_count;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x)
        bounds[open[i].node] = make_float2(open[i].lo, open[i].hi);
}

hipError_t launch_lw_bounds(hipStream_t s, const LWState *st, const LWOpen *open,
                            float2 *bounds) {
    hipLaunchKernelGGL(k_lw_bounds, dim3(1), dim3(256), 0, s, st, open, bounds);
    return hipGetLastError();
}

// The step state the partition plan needs, loaded with the rest of the step
// state when the partition kernel starts.
struct LWPick {
    uint32_t count, child0, leaves, next_slot, dst;
    int32_t node, depth, slot;
};

// Partition plan, run by one block once the left count is known: child
// segments and covers, whether the children are evaluated, histogram slots
// and the smaller child's items (write_items for one pair: same chunking).
// Every thread computes the plan from the preloaded state, so no barrier or
// global read sits between the last cursor add and the item writes; thread 0
// writes the scalar results.
__device__ void lw_plan_block(const Shape &sh, const LWArgs &a, const LWPick &q, LWState *st,
                              LWOpen *open, uint32_t left, uint32_t *slot_seg,
                              uint32_t *slot_count, TreeCtl *ctl, Pair *pairs, HistItem *items,
                              const TreeOut &out) {
    const uint32_t cnt = q.count, right = cnt - left;
    const uint32_t i0 = q.child0, i1 = i0 + 1;
    const int32_t child_depth = q.depth + 1;
    const bool can_eval = child_depth < a.max_depth && (int32_t)q.leaves + 1 < a.num_leaves &&
                          left > 0 && right > 0;
    // the smaller child (ties: left) gets a new slot; the larger one takes
    // over the parent's slot (parent - smaller, in place)
    const bool small_left = left <= right;
    const uint32_t seg_s = small_left ? q.dst : q.dst + left;
    const uint32_t cnt_s = small_left ? left : right;
    const uint32_t T = (uint32_t)sh.hist_tiles;
    const uint32_t chunk =
        can_eval ? item_chunk(cnt_s, 1, sh.hist_tiles, a.target_items, a.min_chunk) : 1u;
    const uint32_t nch = can_eval ? (cnt_s + chunk - 1) / chunk : 0u;
    const uint32_t n_items = nch * T;
    const bool fits = n_items <= sh.item_cap;
    if (threadIdx.x == 0) {
        const int32_t lc = 2 * q.node + 1, rc = lc + 1;
        out.cover[lc] = (float)left;
        out.cover[rc] = (float)right;
        open[i0].seg = q.dst;
        open[i0].count = left;
        open[i1].seg = q.dst + left;
        open[i1].count = right;
        st->left = left;
        st->leaves = q.leaves + 1;
        if (can_eval) {
            const uint32_t s_new = q.next_slot, s_par = (uint32_t)q.slot;
            st->next_slot = s_new + 1;
            const uint32_t is = small_left ? i0 : i1, il = small_left ? i1 : i0;
            open[is].slot = (int32_t)s_new;
            open[il].slot = (int32_t)s_par;
            slot_seg[s_new] = seg_s;
            slot_count[s_new] = cnt_s;
            slot_seg[s_par] = small_left ? q.dst + left : q.dst;
            slot_count[s_par] = cnt - cnt_s;
            st->eval_first = i0;
            st->eval_count = 2;
            Pair p = {};
            p.built = s_new;
            p.derived = s_par;
            p.parent = s_par;
            ctl->chunk = chunk;
            atomicAdd(&ctl->level_built[min(child_depth, 15)], cnt_s);
            ctl->num_pairs = 1;
            if (!fits) {
                // never write past the item list (reported after the tree)
                ctl->num_items = 0;
                ctl->overflow = 1;
            } else {
                p.item_first = 0;
                p.nchunks = nch;
                ctl->num_items = n_items;
            }
            pairs[0] = p;
        } else {
            st->eval_count = 0;
        }
    }
    if (!can_eval || !fits) return;
    for (uint32_t it = threadIdx.x; it < n_items; it += blockDim.x) {
        const uint32_t t = it % T, c = it / T;
        HistItem h;
        h.pair = 0;
        h.tile = t;
        h.start = seg_s + c * chunk;
        h.count = min(chunk, cnt_s - c * chunk);
        items[it] = h;
    }
}

// Partition of the picked leaf's segment into the other half of the order
// buffer, PART_BLOCK entries at a time (grid-stride: the grid is sized for
// the largest segment, the root's, and most steps use a few blocks), lefts
// from the front and rights from the back (route_block).  The block whose
// cursor add reserves the segment's last entries knows the left count from
// that add and runs the plan once its own entries are written; the plan
// reads nothing that another block of this launch writes.
__global__ __launch_bounds__(PART_THREADS, 8) void k_lw_route(Shape sh, LWArgs a, LWState *st,
                                                          LWOpen *open,
                                                          const uint8_t *__restrict__ bins_fm,
                                                          Entry *order, uint64_t *cursor,
                                                          uint32_t *slot_seg, uint32_t *slot_count,
                                                          TreeCtl *ctl, Pair *pairs,
                                                          HistItem *items, TreeOut out) {
    __shared__ uint32_t s_mask[8];
    // the step state, loaded together before any branch
    const uint32_t done = st->done, cnt = st->count, src = st->src, dst = st->dst;
    const NodeSplit sp = {st->feature, st->bin, st->flags};
    const uint32_t mask_word = threadIdx.x < 8 ? st->mask[threadIdx.x] : 0u;
    const LWPick q = {cnt, st->child0, st->leaves, st->next_slot, dst,
                      st->pick_node, st->pick_depth, st->pick_slot};
    if (done) return;
    if (cnt == 0) {                                  // nothing to move: plan directly
        if (blockIdx.x == 0)
            lw_plan_block(sh, a, q, st, open, 0u, slot_seg, slot_count, ctl, pairs, items, out);
        return;
    }
    if (blockIdx.x * (uint32_t)PART_BLOCK >= cnt) return;   // uniform per block
    if (threadIdx.x < 8) s_mask[threadIdx.x] = mask_word;
    __syncthreads();
    const uint8_t *col = bins_fm + (size_t)sp.feature * a.rows;
    bool last = false;
    uint32_t left = 0;
    for (uint32_t first = blockIdx.x * (uint32_t)PART_BLOCK; first < cnt;
         first += gridDim.x * (uint32_t)PART_BLOCK) {
        if (route_block(sp, s_mask, sh.num_bins, col, order + src + first,
                        min((uint32_t)PART_BLOCK, cnt - first), cnt, order + dst, cursor,
                        true, &left))
            last = true;                             // uniform per block
        __syncthreads();                             // LDS reuse by the next chunk
    }
    if (last) lw_plan_block(sh, a, q, st, open, left, slot_seg, slot_count, ctl, pairs, items, out);
}

hipError_t launch_lw_partition(hipStream_t s, const Shape &sh, const LWArgs &a, LWState *st,
                               LWOpen *open, const uint8_t *bins_fm, Entry *order,
                               uint64_t *cursor, uint32_t *slot_seg, uint32_t *slot_count,
                               TreeCtl *ctl, Pair *pairs, HistItem *items, const TreeOut out) {
    hipLaunchKernelGGL(k_lw_route, dim3(a.part_blocks), dim3(PART_THREADS), 0, s, sh, a, st, open,
                       bins_fm, order, cursor, slot_seg, slot_count, ctl, pairs, items, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Leaf-wise growth in depth rounds.  The best-first loop (leaf_pick_apply,
// :720-871) picks, among the open leaves with a valid candidate, the largest
// gain (lowest open index on ties) until the tree has num_leaves leaves.  An
// open leaf Y that n other open leaves beat can only be picked after all of
// them, so it is never picked once n >= the picks left (num_leaves - leaves);
// a node that is not open yet is beaten by every open leaf of equal gain.
// Round r therefore expands (partitions, and builds its children's
// histograms and splits) every evaluated depth-r node that fewer open leaves
// beat than picks are left: a superset of the depth-r leaves the loop will
// pick, and every pick is expanded in the round of its depth.  Each round's
// select kernel replays the loop as far as the expanded nodes allow, so the
// picks, their order and therefore the tree are those of the one-leaf loop.
// Expanded nodes that are never picked cost work, not correctness: their
// splits live only in the speculative tree the partition reads.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int heap_depth(uint32_t n) { return 31 - __clz((int)(n + 1)); }


template <int NW>
__global__ __launch_bounds__(1024) void k_lwb_select(
    Shape sh, SplitParams sp, LWBArgs a, int32_t r, const SplitResult *__restrict__ results,
    uint32_t *count, const int64_t *__restrict__ node_g,
    const int64_t *__restrict__ node_h, float2 *bounds, const int8_t *__restrict__ monotone,
    TreeCtl *ctl, uint64_t *cursors, LWBState *st, SplitResult *cand, TreeOut spec,
    TreeOut out) {
    __shared__ int32_t s_f[LWB_MAX_NODES], s_open[LWB_MAX_NODES];
    __shared__ float s_gain[LWB_MAX_NODES];
    __shared__ uint32_t s_cnt[LWB_MAX_NODES];
    __shared__ float2 s_bounds[LWB_MAX_NODES];
    __shared__ int32_t s_olist[2 * LWB_MAX_LEAVES + 2];
    __shared__ uint32_t s_exp[(LWB_MAX_NODES + 31) / 32];
    __shared__ int32_t s_seq[LWB_MAX_LEAVES];
    __shared__ LWBInfo s_info[LWB_MAX_NODES];
    __shared__ uint32_t s_keys[LWB_MAX_NODES];
    __shared__ int32_t s_rank[LWB_MAX_NODES];
    __shared__ uint2 s_rinfo[LWB_MAX_NODES];
    __shared__ unsigned long long s_omask[NW];
    __shared__ uint32_t s_dup;
    __shared__ uint32_t s_state[5];                  // done, leaves, open count, picks, error
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6, nw = blockDim.x >> 6;
    const int D = a.max_depth, L = a.num_leaves, F = sh.cols;
    const int rr = r < D ? r : D;
    const uint32_t M = (1u << (rr + 1)) - 1u;        // the nodes of depth <= r
    const uint32_t level_start = (1u << rr) - 1u, level_n = 1u << rr;
    const float msg = sp.min_split_gain;
    auto valid = [&](int32_t f, float g) { return f >= 0 && isfinite(g) && g > msg; };
    if (r == 0) {
        // a new tree: every node a leaf of value 0, only the root open
        for (int n = tid; n < a.total_nodes; n += blockDim.x) {
            const NodeSplit leaf = {-1, 0, 0};
            out.split[n] = leaf;
            out.leaf[n] = 0.0f;
            out.gain[n] = 0.0f;
            out.cover[n] = 0.0f;
        }
        for (int k = tid; k < a.total_nodes * 8; k += blockDim.x) out.mask[k] = 0u;
        for (uint32_t w = tid; w < (LWB_MAX_NODES + 31) / 32; w += blockDim.x) s_exp[w] = 0u;
        if (tid == 0) {
            s_f[0] = -1;
            s_gain[0] = -INFINITY;
            s_open[0] = 0;
            s_olist[0] = 0;
            s_cnt[0] = count[0];
            s_bounds[0] = bounds[0];
            s_state[0] = 0; s_state[1] = 1; s_state[2] = 1;
        }
    } else {
        if (tid == 0) {
            s_state[0] = st->done; s_state[1] = st->leaves; s_state[2] = st->open_count;
        }
        for (uint32_t n = tid; n < M; n += blockDim.x) {
            const int32_t f = st->cand_f[n];
            s_f[n] = f;
            s_gain[n] = st->cand_gain[n];
            s_open[n] = st->open[n];
            s_cnt[n] = count[n];
            s_bounds[n] = bounds[n];
        }
        for (uint32_t w = tid; w < (LWB_MAX_NODES + 31) / 32; w += blockDim.x)
            s_exp[w] = st->expanded[w];
    }
    if (tid == 0) { s_state[3] = 0; s_state[4] = 0; }
    __syncthreads();
    const uint32_t oc0 = s_state[2];
    for (uint32_t k = tid; r > 0 && k < oc0; k += blockDim.x) s_olist[k] = st->olist[k];
    auto expanded = [&](uint32_t n) { return ((s_exp[n >> 5] >> (n & 31u)) & 1u) != 0; };
    if (s_state[0]) {
        // finished in an earlier round: nothing of this level is partitioned
        for (uint32_t l = tid; r < D && l < level_n; l += blockDim.x) {
            const NodeSplit leaf = {-1, 0, 0};
            spec.split[level_start + l] = leaf;
        }
        return;                                      // uniform
    }
    const float g_inv = f32_from_bits(ctl->max_gh[0]) / 32767.0f;
    const float h_inv = f32_from_bits(ctl->max_gh[1]) / 127.0f;
    // evaluate the depth-r nodes the last round built: argmax over features
    // (strict '>', lowest feature wins).  A wavefront takes LWB_EVAL nodes at
    // once, their gain loads in flight together; the argmax is two DPP
    // maxima (gain key, then lowest feature).  The candidates themselves are
    // copied with the state write-back.
    for (uint32_t l0 = (uint32_t)wv; r < D && l0 < level_n; l0 += (uint32_t)nw * LWB_EVAL) {
        uint32_t bk[LWB_EVAL], bfe[LWB_EVAL];
        bool ev[LWB_EVAL];
#pragma unroll
        for (int u = 0; u < LWB_EVAL; ++u) {
            const uint32_t l = l0 + (uint32_t)(u * nw);
            ev[u] = l < level_n && (r == 0 || expanded((level_start + l - 1) >> 1));
            bk[u] = 0u;
            bfe[u] = 0u;
        }
        for (int f = lane; f < F; f += 64) {
#pragma unroll
            for (int u = 0; u < LWB_EVAL; ++u) {
                if (!ev[u]) continue;
                const float g = results[(size_t)(l0 + (uint32_t)(u * nw)) * F + f].gain;
                const uint32_t k = g > -INFINITY ? gain_key(g) : 0u;   // NaN, -inf: none
                if (k > bk[u]) { bk[u] = k; bfe[u] = (uint32_t)f; }
            }
        }
#pragma unroll
        for (int u = 0; u < LWB_EVAL; ++u) {
            const uint32_t l = l0 + (uint32_t)(u * nw);
            if (l >= level_n) continue;              // uniform
            const uint32_t n = level_start + l;
            int32_t bf = -1;
            float bg = -INFINITY;
            if (ev[u]) {
                const uint32_t m = wave_max_dpp(bk[u]);
                if (m) {
                    bf = (int32_t)~wave_max_dpp(bk[u] == m ? ~bfe[u] : 0u);
                    bg = key_float(m);
                }
            }
            if (lane == 0) {
                s_f[n] = bf;
                s_gain[n] = bg;
                if (n == 0)                          // the root's own leaf value
                    out.leaf[0] = lw_leaf_value(sp, node_g[0], node_h[0], g_inv, h_inv,
                                                s_bounds[0].x, s_bounds[0].y);
            }
        }
    }
    __syncthreads();
    // Candidate ranks: valid candidates of depth <= r by gain key (largest
    // first, node index on equal keys), 32 comparisons per work item;
    // s_dup marks a repeated key.
    for (uint32_t n = tid; n < M; n += blockDim.x) {
        s_keys[n] = valid(s_f[n], s_gain[n]) ? gain_key(s_gain[n]) : 0u;
        s_rank[n] = 0;
    }
    if (tid < NW) s_omask[tid] = 0ull;
    if (tid == 0) s_dup = 0u;
    __syncthreads();
    {
        constexpr uint32_t RC = 32;
        const uint32_t chunks = (M + RC - 1) / RC;
        for (uint32_t w = tid; w < M * chunks; w += blockDim.x) {
            const uint32_t n = w / chunks, c0 = (w - n * chunks) * RC;
            const uint32_t k = s_keys[n];
            if (!k) continue;
            uint32_t c = 0;
            bool dup = false;
#pragma unroll
            for (uint32_t j = 0; j < RC; ++j) {
                const uint32_t u = c0 + j;
                const uint32_t ku = u < M ? s_keys[u] : 0u;
                c += (ku > k || (ku == k && u < n)) ? 1u : 0u;
                dup |= ku == k && u != n;
            }
            if (c) atomicAdd(&s_rank[n], (int32_t)c);
            if (dup) s_dup = 1u;
        }
    }
    __syncthreads();
    // per rank: node and flags (bit 0 expanded), and the ranks a pick of it
    // opens (0xFFFF: none; children open as candidates when they hold a
    // valid candidate, are not at depth D and both hold rows)
    for (uint32_t n = tid; n < M; n += blockDim.x) {
        if (!s_keys[n]) continue;
        const int32_t rk = s_rank[n];
        uint32_t fl = 0u, rl = 0xFFFFu, rrk = 0xFFFFu;
        if (expanded(n)) {
            const uint32_t lc = 2 * n + 1, rc = lc + 1;
            fl = 1u;
            if (heap_depth(n) + 1 < D && s_cnt[lc] > 0 && s_cnt[rc] > 0) {
                if (lc < M && s_keys[lc]) rl = (uint32_t)s_rank[lc];
                if (rc < M && s_keys[rc]) rrk = (uint32_t)s_rank[rc];
            }
        }
        s_rinfo[rk] = make_uint2(n | (fl << 16), rl | (rrk << 16));
        if (s_open[n] >= 0) atomicOr(&s_omask[rk >> 6], 1ull << (rk & 63));
    }
    __syncthreads();
    // replay the picks (one wavefront; only lane 0 writes LDS in the loops:
    // the open list, for the next rounds and the expansion choice below)
    if (wv == 0) {
        uint32_t leaves = s_state[1], oc = s_state[2], nc = 0, done = 0, err = 0;
        if (!s_dup) {
            // no two candidates share a gain: the pick is the open candidate of
            // lowest rank, the lowest set bit of the open mask (scalar
            // registers); the loop records the picks, the open-list
            // bookkeeping follows them below
            uint64_t mk[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const uint64_t v = s_omask[w];
                mk[w] = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
            }
            for (;;) {
                if ((int)leaves >= L) { done = 1; break; }
                uint32_t p = 0xFFFFFFFFu;
#pragma unroll
                for (int w = NW - 1; w >= 0; --w)
                    if (mk[w]) p = (uint32_t)(w * 64 + __builtin_ctzll(mk[w]));
                if (p == 0xFFFFFFFFu) { done = 1; break; }
                const uint2 q = s_rinfo[p];
                const uint32_t q0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)q.x);
                if (!(q0 & 0x10000u)) {
                    // not partitioned yet: this round's expansion (its depth is r)
                    if (heap_depth(q0 & 0xFFFFu) != rr || r >= D) { err = 1; done = 1; }
                    break;
                }
                const uint32_t q1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)q.y);
                const uint32_t rl = q1 & 0xFFFFu, rrk = q1 >> 16;
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    if ((uint32_t)w == (p >> 6)) mk[w] &= ~(1ull << (p & 63));
                    if ((uint32_t)w == (rl >> 6)) mk[w] |= 1ull << (rl & 63);   // none: no word
                    if ((uint32_t)w == (rrk >> 6)) mk[w] |= 1ull << (rrk & 63);
                }
                if (lane == 0) s_seq[nc] = (int32_t)(q0 & 0xFFFFu);
                leaves += 1;
                nc += 1;
            }
        } else {
            // repeated gains: open entry i lives in lane i % 64, register
            // slot i / 64, as its gain key (0: not a valid candidate) and its
            // node; a pick is the largest key, lowest index on equal keys (two
            // DPP reductions); what a pick needs of its node comes from one
            // LDS record written before the loop.
            for (uint32_t n = (uint32_t)lane; n < M; n += 64) {
                LWBInfo inf = {0u, 0u, 0u, 0u};
                if (expanded(n)) {
                    const uint32_t lc = 2 * n + 1, rc = lc + 1;
                    inf.flags = 1u | ((s_cnt[lc] > 0 && s_cnt[rc] > 0) ? 2u : 0u);
                    inf.kl = valid(s_f[lc], s_gain[lc]) ? gain_key(s_gain[lc]) : 0u;
                    inf.kr = valid(s_f[rc], s_gain[rc]) ? gain_key(s_gain[rc]) : 0u;
                }
                s_info[n] = inf;
            }
            uint32_t ok[LWB_SLOTS];
            int32_t on[LWB_SLOTS];
#pragma unroll
            for (int k = 0; k < LWB_SLOTS; ++k) {
                const uint32_t i = (uint32_t)lane + 64u * k;
                ok[k] = 0u;
                on[k] = 0;
                if (i < oc) {
                    const int32_t n = s_olist[i];
                    on[k] = n;
                    if (s_open[n] == (int32_t)i && valid(s_f[n], s_gain[n]))
                        ok[k] = gain_key(s_gain[n]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            for (;;) {
                if ((int)leaves >= L) { done = 1; break; }
                const uint32_t slots = (oc + 63u) >> 6;   // uniform
                uint32_t bk = 0u, bidx = 0u;
#pragma unroll
                for (int k = 0; k < LWB_SLOTS; ++k)
                    if ((uint32_t)k < slots && ok[k] > bk) { bk = ok[k]; bidx = (uint32_t)lane + 64u * k; }
                const uint32_t m = wave_max_dpp(bk);
                if (m == 0u) { done = 1; break; }
                const uint32_t bi = ~wave_max_dpp(bk == m ? ~bidx : 0u);
                const uint32_t kb = bi >> 6, lb = bi & 63u;
                int32_t xs = on[0];
#pragma unroll
                for (int k = 1; k < LWB_SLOTS; ++k)
                    if ((uint32_t)k == kb) xs = on[k];
                const int32_t x = __builtin_amdgcn_readlane(xs, (int)lb);
                const LWBInfo inf = s_info[x];
                if (!(inf.flags & 1u)) {
                    // not partitioned yet: this round's expansion (its depth is r)
                    if (heap_depth((uint32_t)x) != rr || r >= D) { err = 1; done = 1; }
                    break;
                }
                const bool can_eval = heap_depth((uint32_t)x) + 1 < D && (int)leaves + 1 < L &&
                                      (inf.flags & 2u);
                const uint32_t kl = can_eval ? inf.kl : 0u, kr = can_eval ? inf.kr : 0u;
                const int32_t lc = 2 * x + 1, rc = lc + 1;
                const uint32_t ka = oc >> 6, la_ = oc & 63u, kb2 = (oc + 1) >> 6, lb2 = (oc + 1) & 63u;
#pragma unroll
                for (int k = 0; k < LWB_SLOTS; ++k) {
                    if ((uint32_t)k == kb && (uint32_t)lane == lb) ok[k] = 0u;
                    if ((uint32_t)k == ka && (uint32_t)lane == la_) { ok[k] = kl; on[k] = lc; }
                    if ((uint32_t)k == kb2 && (uint32_t)lane == lb2) { ok[k] = kr; on[k] = rc; }
                }
                if (lane == 0) {
                    if (!can_eval) { s_f[lc] = -1; s_f[rc] = -1; }
                    s_open[x] = -2;
                    s_open[lc] = (int32_t)oc;
                    s_open[rc] = (int32_t)oc + 1;
                    s_olist[oc] = lc;
                    s_olist[oc + 1] = rc;
                    s_seq[nc] = x;
                }
                oc += 2;
                leaves += 1;
                nc += 1;
            }
        }
        if (!s_dup) oc += 2 * nc;                   // two children per pick
        if (lane == 0) {
            s_state[0] = done; s_state[1] = leaves; s_state[2] = oc; s_state[3] = nc;
            s_state[4] = err;
        }
    }
    __syncthreads();
    if (!s_dup) {
        // the fast replay's open-list bookkeeping: pick k appends its children
        // at open entries oc0 + 2k and oc0 + 2k + 1 (children of a pick made
        // with no evaluation left are not candidates), then every pick is
        // marked split (after the appends: a pick may be an earlier child)
        const uint32_t npk = s_state[3], leaves0 = s_state[1] - npk;
        for (uint32_t k = tid; k < npk; k += blockDim.x) {
            const int32_t x = s_seq[k], lc = 2 * x + 1, rc = lc + 1;
            const uint32_t i = oc0 + 2 * k;
            const bool can_eval = heap_depth((uint32_t)x) + 1 < D && (int)(leaves0 + k) + 1 < L &&
                                  s_cnt[lc] > 0 && s_cnt[rc] > 0;
            if (!can_eval) { s_f[lc] = -1; s_f[rc] = -1; }
            s_open[lc] = (int32_t)i;
            s_open[rc] = (int32_t)i + 1;
            s_olist[i] = lc;
            s_olist[i + 1] = rc;
        }
        __syncthreads();
        for (uint32_t k = tid; k < npk; k += blockDim.x) s_open[s_seq[k]] = -2;
        __syncthreads();
    }
    const uint32_t done = s_state[0], leaves = s_state[1], oc = s_state[2], nc = s_state[3];
    // the picks' outputs, parents before children (monotone bounds pass down):
    // split, gain and mask of the picked node, leaf values, bounds and covers
    // of its children (Shaders.swift:1424-1443 for the bounds).  Thread k
    // loads pick k's candidate once; the depth passes read bounds from LDS.
    {
        const bool mine = (uint32_t)tid < nc;
        const int32_t x = mine ? s_seq[tid] : 0;
        SplitResult c = {};
        int64_t G = 0, H = 0;
        int32_t bf = 0;
        int cst = 0;
        if (mine) {
            c = cand[x];
            G = node_g[x];
            H = node_h[x];
            bf = s_f[x];
            cst = (c.flags & FLAG_CATEGORICAL) ? 0 : (int)monotone[bf];
        }
        const int dx = mine ? heap_depth((uint32_t)x) : -1;
        for (int d = 0; d < rr; ++d) {
            if (dx == d) {
                const bool cat = (c.flags & FLAG_CATEGORICAL) != 0;
                const NodeSplit ns = {bf, c.bin, c.flags};
                out.split[x] = ns;
                out.leaf[x] = 0.0f;
                out.gain[x] = c.gain;
                for (int w = 0; w < 8; ++w) out.mask[(size_t)x * 8 + w] = cat ? c.mask[w] : 0u;
                const int64_t lg = c.gl_int, lh = c.hl_int, rg = G - c.gl_int, rh = H - c.hl_int;
                const float2 pb = s_bounds[x];
                float llo = pb.x, lhi = pb.y, rlo = pb.x, rhi = pb.y;
                if (cst != 0) {
                    const float vl = -c.gl / (c.hl + sp.lambda);
                    const float gr = (float)rg * g_inv, hr = (float)rh * h_inv;
                    const float vr = -gr / (hr + sp.lambda);
                    const float mid = clampf(0.5f * (vl + vr), pb.x, pb.y);
                    if (cst > 0) { lhi = fminf(lhi, mid); rlo = fmaxf(rlo, mid); }
                    else { llo = fmaxf(llo, mid); rhi = fminf(rhi, mid); }
                }
                const int32_t lc = 2 * x + 1, rc = lc + 1;
                out.leaf[lc] = lw_leaf_value(sp, lg, lh, g_inv, h_inv, llo, lhi);
                out.leaf[rc] = lw_leaf_value(sp, rg, rh, g_inv, h_inv, rlo, rhi);
                if (!(a.deep_walk && dx + 1 == D)) {     // else counted by the walk
                    out.cover[lc] = (float)s_cnt[lc];
                    out.cover[rc] = (float)s_cnt[rc];
                }
                s_bounds[lc] = make_float2(llo, lhi);
                s_bounds[rc] = make_float2(rlo, rhi);
                bounds[lc] = make_float2(llo, lhi);
                bounds[rc] = make_float2(rlo, rhi);
            }
            __syncthreads();
        }
    }
    if (r == 0 && tid == 0) out.cover[0] = (float)s_cnt[0];
    if (r >= D && a.deep_walk)                       // the walk adds the deepest counts
        for (uint32_t k = tid; k < (1u << D); k += blockDim.x) count[(1u << D) - 1 + k] = 0;
    // the depth-r nodes to expand: evaluated, valid, and beaten by fewer open
    // leaves than picks are left (ballots count the beating entries)
    const int left_picks = L - (int)leaves;
    for (uint32_t l = (uint32_t)wv; r < D && l < level_n; l += (uint32_t)nw) {
        const uint32_t n = level_start + l;
        const int32_t fy = s_f[n];
        const float gy = s_gain[n];
        bool take = false;
        if (!done && valid(fy, gy)) {
            const int32_t oy = s_open[n];
            int beat = 0;
            for (uint32_t i0 = 0; i0 < oc; i0 += 64) {
                const uint32_t i = i0 + (uint32_t)lane;
                bool b = false;
                if (i < oc) {
                    const int32_t z = s_olist[i];
                    if (z != (int32_t)n && s_open[z] == (int32_t)i) {
                        const float gz = s_gain[z];
                        b = valid(s_f[z], gz) &&
                            (gz > gy || (gz == gy && (oy < 0 || (int32_t)i < oy)));
                    }
                }
                beat += __popcll(__ballot(b));
            }
            take = beat < left_picks;
        }
        if (lane == 0) {
            NodeSplit ns = {-1, 0, 0};
            if (take) {
                const SplitResult &c = results[(size_t)l * F + fy];
                ns = NodeSplit{fy, c.bin, c.flags};
                const bool cat = (c.flags & FLAG_CATEGORICAL) != 0;
                for (int w = 0; w < 8; ++w) spec.mask[(size_t)n * 8 + w] = cat ? c.mask[w] : 0u;
                atomicOr(&s_exp[n >> 5], 1u << (n & 31u));
            }
            spec.split[n] = ns;
            cursors[(size_t)l * CURSOR_STRIDE] = 0;  // the level's partition starts at zero
        }
    }
    __syncthreads();
    // keep the state for the next round (a new tree writes every node)
    const uint32_t keep = r == 0 ? (uint32_t)a.total_nodes : M;
    for (uint32_t n = tid; n < keep; n += blockDim.x) {
        st->cand_f[n] = n < M ? s_f[n] : -1;
        st->cand_gain[n] = n < M ? s_gain[n] : -INFINITY;
        st->open[n] = n < M ? s_open[n] : -1;
    }
    for (uint32_t k = tid; k < oc; k += blockDim.x) st->olist[k] = s_olist[k];
    // the evaluated depth-r candidates, a word per thread
    constexpr uint32_t CW = sizeof(SplitResult) / sizeof(uint32_t);
    for (uint32_t k = tid; r < D && k < level_n * CW; k += blockDim.x) {
        const uint32_t l = k / CW, w = k - l * CW, n = level_start + l;
        const int32_t f = s_f[n];
        if (f >= 0)
            reinterpret_cast<uint32_t *>(cand + n)[w] =
                reinterpret_cast<const uint32_t *>(results + (size_t)l * F + f)[w];
    }
    for (uint32_t w = tid; w < (LWB_MAX_NODES + 31) / 32; w += blockDim.x)
        st->expanded[w] = s_exp[w];
    if (tid == 0) {
        st->done = (done || r >= D) ? 1u : 0u;
        st->leaves = leaves;
        st->open_count = oc;
        if (s_state[4]) ctl->overflow = LWB_MISSED_PICK;
    }
}

hipError_t launch_lwb_select(hipStream_t s, const Shape &sh, const SplitParams &sp,
                             const LWBArgs &a, int32_t round, const SplitResult *results,
                             uint32_t *count, const int64_t *node_g, const int64_t *node_h,
                             float2 *bounds, const int8_t *monotone, TreeCtl *ctl,
                             uint64_t *cursors, LWBState *st, SplitResult *cand,
                             const TreeOut spec, const TreeOut out) {
    if (a.max_depth < 1 || a.max_depth > LWB_MAX_DEPTH || a.num_leaves < 2 ||
        a.num_leaves > LWB_MAX_LEAVES || a.total_nodes != (1 << (a.max_depth + 1)) - 1 ||
        round < 0 || round > a.max_depth)
        return hipErrorInvalidValue;
    // the open mask's words: as few as the tree's nodes allow
    const int words = lwb_mask_words(a.max_depth);
#define MBK_LWB_SELECT(W)                                                                     \
    hipLaunchKernelGGL(k_lwb_select<W>, dim3(1), dim3(1024), 0, s, sh, sp, a, round, results, \
                       count, node_g, node_h, bounds, monotone, ctl, cursors, st, cand, spec, out)
    if (words <= 1) MBK_LWB_SELECT(1);
    else if (words <= 2) MBK_LWB_SELECT(2);
    else if (words <= 4) MBK_LWB_SELECT(4);
    else MBK_LWB_SELECT(lwb_mask_words(LWB_MAX_DEPTH));
#undef MBK_LWB_SELECT
    return hipGetLastError();
}

}  // namespace mbk
