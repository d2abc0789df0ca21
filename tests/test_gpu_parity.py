"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Integer/byte work (binning, quantisation, histograms) and the whole trained
model are compared bit for bit; TreeSHAP within 1e-5 relative (+1e-6 abs)
of the oracle's double-precision recursive TreeSHAP.
"""
import ctypes

import numpy as np
import pytest

import dataclasses

import datasets as D
import macboost_amd as mb
import model_io
import oracle_lib as O
from macboost_amd import _core

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = mb.Context(0)
    yield c
    c.close()


def gpu_fit(x_fm, y, params, **kw):
    h = mb.train(params, x_fm, y, feature_major=True, **kw)
    obj = model_io.saved_model(h)
    return h, obj


def oracle_fit(x_fm, y, params, is_cat=None, w=None):
    p = dict(params)
    kw = dict(num_trees=p.pop("num_trees", 100), max_depth=p.pop("max_depth", 6),
              num_leaves=p.pop("num_leaves", 0), learning_rate=p.pop("learning_rate", 0.1),
              lam=p.pop("lambda", 1.0), min_child_hess=p.pop("min_child_weight", 1.0),
              min_split_gain=p.pop("min_split_gain", 0.0), cat_smooth=p.pop("cat_smooth", 10.0))
    nb = p.pop("num_bins", 256)
    obj = p.pop("objective", "regression")
    kw["objective"] = {"regression": O.OBJ_L2, "binary": O.OBJ_LOGISTIC, "mae": O.OBJ_MAE,
                       "quantile": O.OBJ_QUANTILE, "multiclass": O.OBJ_MULTICLASS,
                       "huber": O.OBJ_HUBER, "poisson": O.OBJ_POISSON,
                       "tweedie": O.OBJ_TWEEDIE}[obj]
    if obj == "tweedie":
        kw["aux"] = p.pop("tweedie_variance_power", 1.5)
    if "scale_pos_weight" in p:
        kw["aux"] = p.pop("scale_pos_weight")
    if "feature_fraction" in p:
        kw["feature_fraction"] = p.pop("feature_fraction")
    if "allowed_features" in p:
        kw["allowed_features"] = p.pop("allowed_features")
    if "num_class" in p:
        kw["num_classes"] = p.pop("num_class")
    if "alpha" in p:
        kw["alpha"] = p.pop("alpha")
    mono = p.pop("monotone_constraints", None)
    p.pop("categorical_features", None)
    for key in ("goss", "goss_top_rate", "goss_other_rate", "subsample"):
        if key in p:
            kw[key] = p.pop(key)
    assert not p, p
    return O.fit_raw(x_fm, y, num_bins=nb, is_cat=is_cat, monotone=mono, w=w, **kw)


def check_identical(x_fm, y, params, is_cat=None, x_test=None, w=None):
    h, obj = gpu_fit(x_fm, y, params, sample_weight=w)
    ref = oracle_fit(x_fm, y, params, is_cat, w)
    nodes = ref.forest.nodes_per_tree
    got = model_io.forest_from_json(obj, nodes)
    assert np.float32(obj["baseScore"]) == np.float32(ref.base_score)
    has_cats = is_cat is not None and any(is_cat)
    model_io.assert_same_forest(got, ref.forest, with_cats=has_cats)
    # training predictions: GPU predict on the train matrix == oracle's running
    # preds.  Leaf-wise renewal adds each tree as (preds + first leaf) + change
    # (Booster.swift:1253-1290), which rounds differently from one addition of
    # the final leaf, so there the oracle's own predict is the reference.
    gp_train = mb.predict(h, x_fm, feature_major=True)
    if params.get("objective") in ("poisson", "tweedie"):
        # log link: predict returns exp(raw score) (Booster.swift:1992-1997);
        # the raw scores are the oracle's running predictions
        assert np.allclose(gp_train, np.exp(ref.preds.astype(np.float64)), rtol=2e-7, atol=0)
        if x_test is not None:
            gp = mb.predict(h, x_test, feature_major=True)
            cp = O.predict(ref.forest, ref.base_score, ref.num_bins, x_test)
            assert np.allclose(gp, np.exp(cp.astype(np.float64)), rtol=2e-7, atol=0)
        return h, ref
    if params.get("num_leaves", 0) > 0 and params.get("objective") in ("mae", "quantile"):
        assert np.array_equal(gp_train, O.predict(ref.forest, ref.base_score, ref.num_bins, x_fm))
        assert np.allclose(gp_train, ref.preds, rtol=1e-5, atol=1e-4)
    else:
        assert np.array_equal(gp_train, ref.preds)
    if x_test is not None:
        gp = mb.predict(h, x_test, feature_major=True)
        cp = O.predict(ref.forest, ref.base_score, ref.num_bins, x_test)
        assert np.array_equal(gp, cp)
    return h, ref


# --------------------------------------------------------------------------
# kernel seam (mbk_*)
# --------------------------------------------------------------------------

def _edge_columns(rows, seed):
    # Columns that stress the sort: NaN holes, heavy ties, +-0 and +-inf,
    # negatives, an all-NaN column, a categorical column, a constant column.
    rng = np.random.default_rng(seed)
    x = np.empty((9, rows), np.float32)
    x[0] = rng.standard_normal(rows)
    x[1] = rng.uniform(-1, 1, rows)
    x[1, rng.random(rows) < 0.3] = np.nan
    x[2] = np.floor(rng.uniform(-5, 5, rows))                 # 10 distinct values
    x[3] = rng.choice(np.array([-0.0, 0.0, 1.0, -np.inf, np.inf, -2.5], np.float32), rows)
    x[4] = np.nan
    x[5] = np.floor(rng.uniform(0, 30, rows))                 # categorical
    x[6] = 7.25
    x[7] = rng.exponential(1.0, rows) * np.where(rng.random(rows) < 0.5, -1e30, 1e-30)
    x[8] = (rng.standard_normal(rows) * 1e-38).astype(np.float32)   # subnormals
    is_cat = np.zeros(9, np.uint8)
    is_cat[5] = 1
    return x, is_cat


@pytest.mark.parametrize("rows,nb,row_major", [(1, 4, False), (777, 64, False),
                                               (5003, 256, True), (200_001, 256, False),
                                               (2_500_003, 255, True)])
def test_quantile_edges_match_oracle(ctx, rows, nb, row_major):
    # computeEdges (Binner.swift:25-56): step 1 below 400k rows, then a
    # stride subsample; equal as floats (a +0/-0 tie may pick either zero).
    x, is_cat = _edge_columns(rows, rows)
    want = O.compute_edges(x, nb, is_cat)
    cols = x.shape[0]
    if row_major:
        dx, rs, cs = ctx.upload(np.ascontiguousarray(x.T)), cols, 1
    else:
        dx, rs, cs = ctx.upload(x), 1, rows
    dc, de = ctx.upload(is_cat), ctx.alloc(cols * (nb - 2) * 4)
    err = ctypes.c_char_p()
    rc = _core.lib().mbk_quantile_edges(ctx.ptr, dx, rows, cols, rs, cs, nb, dc, de,
                                        ctypes.byref(err))
    assert rc == 0, err.value
    got = ctx.download(de, (cols, nb - 2), np.float32)
    assert np.array_equal(got, want)
    s = got[[0, 1, 2, 3, 7, 8]]
    assert (s[:, 1:] >= s[:, :-1]).all()                     # sorted (infs included)
    assert not got[[4, 5]].any()


@pytest.mark.parametrize("tile_w", [8, 16, 32, 64])
def test_bin_data_matches_oracle(ctx, tile_w):
    rows, cols, nb = 5003, 37, 256
    x, _ = O.friedman(rows, cols, 3)
    x[2, ::7] = np.nan
    x[5] = np.floor(x[5] * 40)
    is_cat = np.zeros(cols, np.uint8)
    is_cat[5] = 1
    e = O.compute_edges(x, nb, is_cat)
    want = O.bin_matrix(x, e, nb, is_cat)
    T = (cols + tile_w - 1) // tile_w
    dx, de, dc = ctx.upload(x), ctx.upload(e), ctx.upload(is_cat)
    dt, df = ctx.alloc(T * rows * tile_w), ctx.alloc(cols * rows)
    err = ctypes.c_char_p()
    rc = _core.lib().mbk_bin_data(ctx.ptr, dx, rows, cols, 1, rows, de, dc, nb, tile_w, dt, df,
                                  ctypes.byref(err))
    assert rc == 0, err.value
    fm = ctx.download(df, (cols, rows), np.uint8)
    tiled = ctx.download(dt, (rows, T, tile_w), np.uint8)
    assert np.array_equal(fm, want)
    for f in range(cols):
        assert np.array_equal(tiled[:, f // tile_w, f % tile_w], want[f])
    pad = T * tile_w - cols
    if pad:
        assert not tiled[:, T - 1, tile_w - pad:].any()


@pytest.mark.parametrize("objective,offset", [(O.OBJ_L2, 0), (O.OBJ_LOGISTIC, 0),
                                              (O.OBJ_LOGISTIC, 1)])
def test_quantize_matches_oracle(ctx, objective, offset):
    # offset 1: inputs start one float past a 16-byte boundary (no vector loads)
    rng = np.random.default_rng(9)
    n = 40_003
    preds = rng.normal(size=n + 1).astype(np.float32)
    y = (rng.random(n + 1) < 0.4).astype(np.float32) if objective == O.OBJ_LOGISTIC else \
        rng.normal(size=n + 1).astype(np.float32)
    w = rng.random(n + 1).astype(np.float32)
    g, h, mg, mh = O.gradients(preds[offset:offset + n], y[offset:offset + n],
                               w[offset:offset + n], objective=objective, aux=1.5)
    want = O.quantize(g, h, mg, mh)
    dp, dy, dw = (ctx.upload(a) + 4 * offset for a in (preds, y, w))
    dm, de = ctx.alloc(8), ctx.alloc(8 * n)
    err = ctypes.c_char_p()
    rc = _core.lib().mbk_quantize(ctx.ptr, objective, 0.9, 1.5, dp, dy, dw, n, dm, de,
                                  ctypes.byref(err))
    assert rc == 0, err.value
    m = ctx.download(dm, 2, np.uint32)
    assert m.view(np.float32).tolist() == [mg, mh]
    ent = ctx.download(de, (n, 2), np.uint32)
    assert np.array_equal(ent[:, 0], np.arange(n))
    assert np.array_equal(ent[:, 1], want)


# 32-wide tiles whose last tile holds few features fold them into the other
# tiles' items (Shape::extras): 34 columns = one item with 2 extras, 65 = (1, 0),
# 99 = (1, 1, 1), 100 = (2, 1, 1); 45 keeps a tile of its own.
@pytest.mark.parametrize("tile_w,nb,n,cols", [(8, 256, 70_000, 45), (32, 64, 150_001, 45),
                                              (64, 256, 2500, 45), (16, 17, 9000, 45),
                                              (32, 256, 150_001, 100), (32, 64, 70_000, 34),
                                              (32, 256, 20_000, 65), (32, 17, 5000, 99)])
def test_node_hist_and_splits_match_oracle(ctx, tile_w, nb, n, cols):
    rng = np.random.default_rng(tile_w + nb + cols)
    rows = 200_000
    bins = rng.integers(0, nb, size=(cols, rows)).astype(np.uint8)
    bins[3, rng.random(rows) < 0.3] = nb - 1              # missing values
    bins[4] = rng.integers(0, 5, size=rows)               # low-cardinality categorical
    bins[4, rng.random(rows) < 0.1] = nb - 1
    is_cat = np.zeros(cols, np.uint8)
    is_cat[4] = 1
    mono = np.zeros(cols, np.int8)
    mono[7], mono[8] = 1, -1
    qg = rng.integers(-32767, 32768, size=rows)
    qh = rng.integers(0, 128, size=rows)
    ghq = (((qg & 0xFFFF).astype(np.uint32) << 16) | qh.astype(np.uint32)).astype(np.uint32)
    idx = np.sort(rng.choice(rows, n, replace=False)).astype(np.uint32)
    T = (cols + tile_w - 1) // tile_w
    tiled = np.zeros((rows, T, tile_w), np.uint8)
    for f in range(cols):
        tiled[:, f // tile_w, f % tile_w] = bins[f]
    ent = np.stack([idx, ghq[idx]], axis=1).astype(np.uint32)
    max_g, max_h = np.float32(3.5), np.float32(0.25)
    mgh = np.array([max_g, max_h], np.float32).view(np.uint32)
    dt, de, dm = ctx.upload(tiled), ctx.upload(ent), ctx.upload(mgh)
    dc, dmo = ctx.upload(is_cat), ctx.upload(mono)
    dh = ctx.alloc(cols * nb * 2 * 8)
    dr = ctx.alloc(cols * 72)
    err = ctypes.c_char_p()
    lam, mch, sm = 1.0, 1.0, 10.0
    rc = _core.lib().mbk_node_hist_split(ctx.ptr, dt, rows, cols, nb, tile_w, de, n, dm, dc, dmo,
                                         lam, mch, sm, dh, dr, ctypes.byref(err))
    assert rc == 0, err.value
    hist = ctx.download(dh, (nb, cols, 2), np.int64)
    hg, hh = O.hist_node(bins, nb, ghq, idx)
    assert np.array_equal(hist[:, :, 0].T, hg) and np.array_equal(hist[:, :, 1].T, hh)
    raw = ctx.download(dr, (cols, 72), np.uint8)
    g_inv, h_inv = np.float32(max_g / np.float32(32767)), np.float32(max_h / np.float32(127))
    G, H = int(hg[0].sum()), int(hh[0].sum())
    for f in range(cols):
        r = O.find_split(hg[f], hh[f], is_cat[f], int(mono[f]), G, H, g_inv, h_inv, lam, mch, sm)
        gain = raw[f, 0:4].view(np.float32)[0]
        b, fl = raw[f, 4:8].view(np.uint32)[0], raw[f, 16:20].view(np.uint32)[0]
        gl, hl = raw[f, 8:12].view(np.float32)[0], raw[f, 12:16].view(np.float32)[0]
        gli, hli = raw[f, 24:32].view(np.int64)[0], raw[f, 32:40].view(np.int64)[0]
        assert np.float32(r.gain).tobytes() == gain.tobytes(), f
        if np.isfinite(r.gain):
            assert (b, fl, gli, hli) == (r.bin, r.flags, r.gl_int, r.hl_int), f
            assert gl == np.float32(r.gl) and hl == np.float32(r.hl), f
            if is_cat[f]:
                mask = raw[f, 40:72].view(np.uint32)
                order = O.cat_order(hg[f], hh[f], g_inv, h_inv, sm)
                want = np.zeros(8, np.uint32)
                for c in order[: r.bin]:
                    want[c >> 5] |= np.uint32(1) << np.uint32(c & 31)
                assert np.array_equal(mask, want), f


def test_node_hist_full_size_exact(ctx):
    # 26M rows x 100 features (two 64-wide tiles), a node holding 4 of every
    # 5 rows: more items than one round of the grid, so the level is cut into
    # several rounds of chunks.  Every feature's bins sum to the node totals
    # (a checksum of checksums), and features at the tile edges match
    # numpy's weighted bincount exactly.
    rows, cols, nb, W = 26_000_000, 100, 256, 64
    rng = np.random.default_rng(2024)
    tiled = np.frombuffer(rng.bytes(2 * rows * W), np.uint8).reshape(rows, 2, W)
    idx = np.flatnonzero(np.arange(rows) % 5 != 0).astype(np.uint32)
    n = idx.size
    qg = rng.integers(-32767, 32768, size=n)
    qh = rng.integers(0, 128, size=n)
    ghq = (((qg & 0xFFFF).astype(np.uint32) << 16) | qh.astype(np.uint32)).astype(np.uint32)
    ent = np.stack([idx, ghq], axis=1)
    mgh = np.array([1.0, 1.0], np.float32).view(np.uint32)
    dt, de, dm = ctx.upload(tiled), ctx.upload(ent), ctx.upload(mgh)
    del ent
    dh = ctx.alloc(cols * nb * 2 * 8)
    dr = ctx.alloc(cols * 72)
    err = ctypes.c_char_p()
    rc = _core.lib().mbk_node_hist_split(ctx.ptr, dt, rows, cols, nb, W, de, n, dm, None, None,
                                         1.0, 1.0, 10.0, dh, dr, ctypes.byref(err))
    assert rc == 0, err.value
    hist = ctx.download(dh, (nb, cols, 2), np.int64)
    assert (hist[:, :, 0].sum(axis=0) == int(qg.sum())).all()
    assert (hist[:, :, 1].sum(axis=0) == int(qh.sum())).all()
    for f in (0, 31, 32, 63, 64, 95, 96, 99):
        b = tiled[idx, f // W, f % W]
        assert np.array_equal(hist[:, f, 0], np.bincount(b, weights=qg, minlength=nb).astype(np.int64)), f
        assert np.array_equal(hist[:, f, 1], np.bincount(b, weights=qh, minlength=nb).astype(np.int64)), f


class _SeamTree:
    """Device buffers of a level-wise tree grown through the mbk_* seam alone."""

    def __init__(self, ctx, x_fm, is_cat, nb, tile_w, depth):
        cols, rows = x_fm.shape
        self.ctx, self.rows, self.cols, self.nb, self.D = ctx, rows, cols, nb, depth
        T = (cols + tile_w - 1) // tile_w
        nodes, lvl = 2 ** (depth + 1) - 1, 2 ** (depth - 1)
        self.nodes = nodes
        self.x = ctx.upload(x_fm)
        self.is_cat = ctx.upload(np.asarray(is_cat, np.uint8))
        self.edges = ctx.alloc(cols * (nb - 2) * 4)
        ctx.call("mbk_quantile_edges", self.x, rows, cols, 1, rows, nb, self.is_cat, self.edges)
        self.tiled, self.fm = ctx.alloc(rows * T * tile_w), ctx.alloc(rows * cols)
        ctx.call("mbk_bin_data", self.x, rows, cols, 1, rows, self.edges, self.is_cat, nb, tile_w,
                 self.tiled, self.fm)
        self.ent = [ctx.alloc(rows * 8), ctx.alloc(rows * 8)]
        self.hist = [ctx.alloc(lvl * nb * cols * 16), ctx.alloc(lvl * nb * cols * 16)]
        self.results, self.max_gh = ctx.alloc(lvl * cols * 72), ctx.alloc(8)
        self.shape = _core.MbkTreeShape(rows, cols, nb, tile_w, depth)
        self.sp = _core.MbkSplitParams(1.0, 1.0, 0.0, 10.0, 0.1)

    def out(self):
        c, n = self.ctx, self.nodes
        o = _core.MbkTreeOut(c.alloc(n * 12), c.alloc(n * 4), c.alloc(n * 4), c.alloc(n * 4),
                             c.alloc(n * 32))
        return o

    def read(self, o):
        c, n = self.ctx, self.nodes
        split = c.download(o.split, (n, 3), np.int32)
        return {"feature": split[:, 0], "bin": split[:, 1].view(np.uint32),
                "flags": split[:, 2].view(np.uint32), "leaf": c.download(o.leaf, n, np.float32),
                "gain": c.download(o.gain, n, np.float32),
                "cover": c.download(o.cover, n, np.float32),
                "mask": c.download(o.mask, (n, 8), np.uint32)}


def _assert_tree_equals_oracle(got, ref, t, edges, nb):
    f = ref.forest
    assert np.array_equal(got["feature"], f.feature[t])
    split = got["feature"] >= 0
    assert np.array_equal(got["bin"][split], f.split_bin[t][split])
    assert np.array_equal(got["flags"][split], f.flags[t][split])
    for name in ("leaf", "gain", "cover"):
        assert np.array_equal(got[name], getattr(f, name)[t]), name
    if f.cat_mask is not None:
        assert np.array_equal(got["mask"], f.cat_mask[t])
    # thresholds come from the edges: edges[f * (nb - 2) + bin] for numeric splits
    num = split & ((got["flags"] & O.FLAG_CATEGORICAL) == 0)
    thr = edges.reshape(-1)[got["feature"][num] * (nb - 2) + got["bin"][num]]
    assert np.array_equal(thr, f.threshold[t][num])


@pytest.mark.parametrize("shape", ["mixed", "wide", "wide32"])
def test_trees_grown_through_the_seam_equal_the_oracle(ctx, shape):
    # fitImpl's level loop on the kernel seam alone (Booster.swift:1467-1648):
    # quantile edges, binning, then per tree quantise -> begin -> per level
    # hist_build, hist_subtract, find_splits, decide_level, route -> final
    # leaves; every tree array equals the oracle's, and so do the running
    # predictions.  Then mbk_grow_tree (the same in one call) and mbk_treeshap.
    if shape == "mixed":
        x, y = _mixed(12_000)
        is_cat, nb, tile_w, depth = [0] * 6 + [1], 64, 8, 5
        mono = np.array([0, 0, 0, 1, 0, 0, 0], np.int8)
    else:
        # wide32: 32-wide tiles, the last tile's 4 features folded into the others
        x, y = mb.friedman(60_000, 100, 17)
        is_cat, nb, tile_w, depth = [0] * 100, 256, (64 if shape == "wide" else 32), 6
        mono = np.zeros(100, np.int8)
    cols, rows = x.shape
    trees = 3
    ref = O.fit_raw(x, y, num_bins=nb, is_cat=is_cat, monotone=mono, num_trees=trees,
                    max_depth=depth)
    st = _SeamTree(ctx, x, is_cat, nb, tile_w, depth)
    edges = ctx.download(st.edges, (cols, nb - 2), np.float32)
    assert np.array_equal(edges, O.compute_edges(x, nb, is_cat))
    labels = ctx.upload(y)
    d_mono = ctx.upload(mono)
    for one_call in (False, True):
        preds = ctx.upload(np.full(rows, np.float32(ref.base_score), np.float32))
        for t in range(trees):
            o = st.out()
            ctx.call("mbk_quantize", 0, 0.9, 0.0, preds, labels, None, rows, st.max_gh, st.ent[0])
            if one_call:
                ctx.call("mbk_grow_tree", ctypes.byref(st.shape), ctypes.byref(st.sp), st.tiled,
                         st.fm, st.is_cat, d_mono, None, st.max_gh, st.ent[0], st.ent[1], rows,
                         st.hist[0], st.hist[1], st.results, o, preds)
            else:
                ctx.call("mbk_tree_begin", ctypes.byref(st.shape), st.max_gh, rows, o)
                with pytest.raises(mb.MacBoostError, match="out of order"):
                    ctx.call("mbk_hist_build", 1, st.tiled, st.ent[0], st.hist[0])
                for d in range(depth):
                    cur, nxt = d % 2, 1 - d % 2
                    ctx.call("mbk_hist_build", d, st.tiled, st.ent[cur], st.hist[cur])
                    ctx.call("mbk_hist_subtract", d, st.hist[nxt], st.hist[cur])
                    ctx.call("mbk_find_splits", d, st.hist[cur], st.is_cat, d_mono, None,
                             ctypes.byref(st.sp), st.results)
                    ctx.call("mbk_decide_level", d, st.results, d_mono, ctypes.byref(st.sp), o)
                    ctx.call("mbk_route", d, st.fm, st.ent[cur], st.ent[nxt], o)
                ctx.call("mbk_final_leaves", st.fm, ctypes.byref(st.sp), o, preds)
            _assert_tree_equals_oracle(st.read(o), ref, t, edges, nb)
        assert np.array_equal(ctx.download(preds, rows, np.float32), ref.preds)
    # TreeSHAP of device rows under the oracle's forest (host arrays)
    f = ref.forest
    n = min(rows, 3000)
    xs = np.ascontiguousarray(x[:, :n])
    d_xs, d_out = ctx.upload(xs), ctx.alloc(n * (cols + 1) * 4)
    mask = np.ascontiguousarray(f.cat_mask) if f.cat_mask is not None else None
    ctx.call("mbk_treeshap", f.feature.ctypes.data, f.threshold.ctypes.data,
             f.flags.ctypes.data, f.leaf.ctypes.data, f.cover.ctypes.data,
             None if mask is None else mask.ctypes.data, f.num_trees, f.nodes_per_tree,
             ref.base_score, nb - 1, d_xs, n, cols, d_out)
    got = ctx.download(d_out, (n, cols + 1), np.float32)
    assert np.allclose(got, O.treeshap(f, ref.base_score, nb, xs), rtol=1e-5, atol=1e-6)


def test_fit_from_device_features_equals_macboost_train(ctx):
    # mbk_fit: the whole fit over raw features already in HBM gives the
    # model macboost_train gives from host memory, in both layouts, with the
    # same warnings and the same categorical error
    rows = 9000
    x, y = _mixed(rows)
    x = x.copy()
    x[3] = y + np.float32(0.0)                       # leakage warning
    params = {"num_trees": 12, "max_depth": 5, "categorical_features": [6]}
    want_h = mb.train(params, x, y, feature_major=True)
    want = model_io.saved_model(want_h)
    for row_major in (False, True):
        d = ctx.upload(np.ascontiguousarray(x.T) if row_major else x)
        h = ctx.fit(params, d, rows, 7, y, row_major=row_major)
        assert model_io.saved_model(h) == want
        assert mb.warnings(h) == mb.warnings(want_h)
        assert any("correlates with the label" in w for w in mb.warnings(h))
    xv, yv = _mixed(2000, 213, 214)
    h = ctx.fit(dict(params, early_stopping_rounds=3), ctx.upload(x), rows, 7, y,
                eval_set=(xv.T, yv))
    h2 = mb.train(dict(params, early_stopping_rounds=3), x, y, eval_set=(xv.T, yv),
                  feature_major=True)
    assert model_io.saved_model(h) == model_io.saved_model(h2)
    assert np.array_equal(mb.eval_history(h), mb.eval_history(h2))
    bad = x.copy()
    bad[6, 4321] = 300.0
    bad[6, 5000] = -1.0
    with pytest.raises(mb.MacBoostError) as e1:
        ctx.fit(params, ctx.upload(bad), rows, 7, y)
    with pytest.raises(mb.MacBoostError) as e2:
        mb.train(params, bad, y, feature_major=True)
    assert str(e1.value) == str(e2.value)
    assert "Categorical feature 6 has value 300.0" in str(e1.value)


# --------------------------------------------------------------------------
# whole fits: identical trees, bit-exact predictions
# --------------------------------------------------------------------------

def test_c1_friedman_identical_trees_and_bitexact_predict():
    # The small Friedman #1 workload: 20k x 100, max_bin 64, 100 trees, depth 6,
    # lr 0.1; held-out 20k rows predicted bit-exactly.
    x, y = mb.friedman(20_000, 100, 42)
    xt, _ = mb.friedman(20_000, 100, 42 + 999)
    check_identical(x, y, {"num_trees": 100, "max_depth": 6, "num_bins": 64}, x_test=xt)


def test_nan_and_categorical_identical_trees():
    rows = 30_000
    x, y = O.friedman(rows, 10, 21)
    rng = O.SplitMix(22)
    miss = O.SplitMix(23).uniforms(5 * rows).reshape(5, rows) < 0.2
    x[:5][miss] = np.nan
    cat = np.array([rng.next() % 13 for _ in range(rows)], np.float32)
    cat[::17] = np.nan
    x = np.vstack([x, cat[None, :]])
    y = (y + np.where(cat % 4 == 1, 3.0, 0.0)).astype(np.float32)
    is_cat = [0] * 10 + [1]
    params = {"num_trees": 30, "max_depth": 6, "num_bins": 256, "categorical_features": [10]}
    xt = x[:, :5000].copy()
    xt[10, :50] = 200.0                                   # unseen category -> missing
    h, ref = check_identical(x, y, params, is_cat=is_cat, x_test=xt)
    assert (ref.forest.flags & O.FLAG_CATEGORICAL).any()
    assert (ref.forest.flags & O.FLAG_DEFAULT_LEFT).any()


def test_logistic_and_monotone_identical_trees():
    rows = 20_000
    rng = O.SplitMix(3)
    x = rng.uniforms(rows * 4).reshape(4, rows)
    y = np.array([1.0 if (x[0, i] + x[1, i] + np.float32(0.3) * np.float32(rng.normal())) > 1
                  else 0.0 for i in range(rows)], np.float32)
    check_identical(x, y, {"num_trees": 30, "max_depth": 5, "objective": "binary"})
    xr, yr = O.friedman(15_000, 6, 101)
    check_identical(xr, yr, {"num_trees": 30, "max_depth": 6,
                             "monotone_constraints": [0, 0, 0, 1, 0, -1]})


def test_reference_known_answers_on_gpu():
    # MacBoostTests.swift:54-70
    h, _ = gpu_fit(np.array([[0, 0, 1, 1]], np.float32), np.array([0, 0, 10, 10], np.float32),
                   {"num_trees": 1, "max_depth": 1, "learning_rate": 0.1, "lambda": 0.0})
    p = mb.predict(h, np.array([[0, 1]], np.float32), feature_major=True)
    assert p[0] == pytest.approx(4.5, abs=1e-4) and p[1] == pytest.approx(5.5, abs=1e-4)
    # FeatureTests.swift:19-38
    for joins_zero in (True, False):
        x = np.array([[0.0] * 100 + [1.0] * 100 + [np.nan] * 100], np.float32)
        y = np.array([10.0] * 100 + [0.0] * 100 + [10.0 if joins_zero else 0.0] * 100, np.float32)
        h, _ = gpu_fit(x, y, {"num_trees": 30, "max_depth": 1, "learning_rate": 0.3})
        p = mb.predict(h, np.array([[0.0, 1.0, np.nan]], np.float32), feature_major=True)
        assert p.tolist() == pytest.approx([10, 0, 10 if joins_zero else 0], abs=0.2)
    # MacBoostTests.swift:185-211: min_child_weight blocks all splits; constant labels
    x, y = O.friedman(5000, 6, 6)
    _, obj = gpu_fit(x, y, {"num_trees": 5, "max_depth": 6, "min_child_weight": 5001.0})
    assert all(t["feature"][0] == -1 for t in obj["trees"])
    h, obj = gpu_fit(x, np.full(5000, 3.25, np.float32), {"num_trees": 10, "max_depth": 5})
    assert np.all(np.abs(mb.predict(h, x, feature_major=True) - 3.25) < 1e-4)


@pytest.mark.parametrize("min_split_gain", [0.0, 40.0])
def test_levelwise_equal_gains_and_min_split_gain_identical(min_split_gain):
    # Duplicated columns give every node's split search exactly equal gains on
    # two or three features (numeric with NaN holes, and categorical): the
    # level's decision must take the lowest feature, as decide_splits' argmax
    # does.  A positive min_split_gain turns nodes whose best gain falls below
    # it into leaves at every level (checked against the oracle in every array).
    rng = np.random.default_rng(77)
    n = 9000
    base = rng.random((3, n), dtype=np.float32)
    base[1, rng.random(n) < 0.15] = np.nan
    cat = rng.integers(0, 9, n).astype(np.float32)
    x = np.stack([base[0], base[1], cat, base[0], base[2], base[1], cat, base[0]])
    y = (10 * base[0] + 5 * np.nan_to_num(base[1], nan=0.7) + (cat % 3) * 2
         + rng.standard_normal(n)).astype(np.float32)
    params = {"num_trees": 8, "max_depth": 6, "num_bins": 64,
              "categorical_features": [2, 6], "min_split_gain": min_split_gain}
    _, ref = check_identical(np.ascontiguousarray(x), y, params, is_cat=[0, 0, 1, 0, 0, 0, 1, 0])
    used = set(int(f) for f in ref.forest.feature.ravel() if f >= 0)
    assert used and used <= {0, 1, 2, 4}              # never a later copy
    if min_split_gain > 0:
        # nodes stop early: fewer splits than the same trees without the floor
        free = oracle_fit(np.ascontiguousarray(x), y, dict(params, min_split_gain=0.0),
                          [0, 0, 1, 0, 0, 0, 1, 0])
        assert (ref.forest.feature >= 0).sum() < (free.forest.feature >= 0).sum()


def test_depth_extremes_identical():
    x, y = O.friedman(3000, 5, 221)
    check_identical(x, y, {"num_trees": 4, "max_depth": 12, "num_bins": 32})
    check_identical(x, y, {"num_trees": 10, "max_depth": 1, "num_bins": 4})


@pytest.mark.parametrize("depth,objective", [(2, "regression"), (3, "regression"), (3, "huber"),
                                             (4, "mae"), (5, "regression")])
def test_shallow_levelwise_partitions_identical(depth, objective):
    # Unsampled, unweighted trees with h = 1 for every row: the root partition
    # writes only its built child's entries, the level-1 partition (depth >= 3)
    # takes every row from the root's implicit words, and the partition before
    # the deepest split level writes only the children that level builds.
    # Categorical and NaN-holed columns at the root and level 1; a row count
    # of many partition blocks that is not a multiple of 64.
    rng = np.random.default_rng(depth * 31 + len(objective))
    n = 150_001
    num = rng.random((5, n), dtype=np.float32)
    num[rng.random((5, n)) < 0.1] = np.nan
    cat = rng.integers(0, 20, (2, n)).astype(np.float32)
    x = np.ascontiguousarray(np.concatenate([num[:3], cat[:1], num[3:], cat[1:]]))
    y = (4 * np.nan_to_num(num[0], nan=0.3) + 1.5 * (cat[0] % 4) + 2 * np.nan_to_num(num[1])
         + (cat[1] % 3) + rng.standard_normal(n)).astype(np.float32)
    params = {"num_trees": 4, "max_depth": depth, "num_bins": 64, "objective": objective,
              "categorical_features": [3, 6]}
    if objective == "huber":
        params["alpha"] = 1.0
    _, ref = check_identical(x, y, params, is_cat=[0, 0, 0, 1, 0, 0, 1])
    # both a categorical and a numeric split among the root and level-1 splits
    top = ref.forest.feature[:, :3].ravel()
    assert set(int(f) for f in top if f >= 0) & {3, 6}
    assert set(int(f) for f in top if f >= 0) - {3, 6}


@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 3), (5, 9), (63, 17), (64, 33), (65, 65),
                                       (130, 100), (8193, 4)])
def test_tiny_and_ragged_shapes_identical(rows, cols):
    # rows below, at and past one wavefront and one partition block; every
    # tile width (8/16/32/64) with partial last tiles; NaN holes
    rng = np.random.default_rng(rows * 1000 + cols)
    x = rng.random((cols, rows), dtype=np.float32)
    x[rng.random((cols, rows)) < 0.1] = np.nan
    y = (rng.standard_normal(rows) + 3.0 * np.nan_to_num(x[0])).astype(np.float32)
    xt = rng.random((cols, 97), dtype=np.float32)
    p = {"num_trees": 4, "max_depth": 6, "num_bins": 32, "min_child_weight": 0.5}
    check_identical(x, y, p, x_test=xt)
    check_identical(x, y, dict(p, num_leaves=5), x_test=xt)


def test_save_load_bitwise(tmp_path):
    # FeatureTests.swift:307-341
    x, y = _mixed(8000)
    h, _ = gpu_fit(x, y, {"num_trees": 20, "max_depth": 5, "categorical_features": [6]})
    mb.save(h, tmp_path / "m.json")
    h2 = mb.load(tmp_path / "m.json")
    assert np.array_equal(mb.predict(h, x, feature_major=True),
                          mb.predict(h2, x, feature_major=True))


def test_leakage_and_bin_hint_warnings():
    # Booster.swift:1771-1808 (a feature that is the label) and :730-738
    # (10,000 rows at 256 bins: 39 rows per bin), in that order
    rng = np.random.default_rng(7)
    x = rng.random((6, 10_000), dtype=np.float32)
    y = rng.standard_normal(10_000).astype(np.float32)
    x[3] = y
    h = mb.train({"num_trees": 2, "max_depth": 3}, x, y, feature_major=True)
    w = mb.warnings(h)
    assert len(w) == 2
    assert "feature 3 correlates with the label" in w[0]
    assert w[1].startswith("max_bin=256 gives ~39 rows per bin")


# --------------------------------------------------------------------------
# benchmark configurations (tree counts bounded by the oracle's speed)
# --------------------------------------------------------------------------

def test_c2_friedman_1m_identical_trees():
    # Friedman #1 at 1M x 100, 256 bins, depth 6; 200k held-out rows
    x, y = mb.friedman(1_000_000, 100, 42)
    xt, _ = mb.friedman(200_000, 100, 42 + 999)
    check_identical(x, y, {"num_trees": 4, "max_depth": 6, "num_bins": 256}, x_test=xt)


def test_c3_nan_categorical_identical_trees():
    # Friedman #1 with 20% MCAR NaN over the numeric columns and 20 integer
    # categorical columns
    x, y, cats = D.c3_mixed(300_000, 42)
    xv, _, _ = D.c3_mixed(50_000, 42 + 999)
    h, ref = check_identical(x, y, {"num_trees": 5, "max_depth": 6, "categorical_features": cats},
                             is_cat=[0] * 80 + [1] * 20, x_test=xv)
    assert (ref.forest.flags & O.FLAG_CATEGORICAL).any()


def test_c4_higgs_like_logistic_identical_trees():
    # 28 HIGGS-shaped synthetic features, logistic objective
    x, y = D.c4_higgs_like(200_000, 42)
    xt, _ = D.c4_higgs_like(50_000, 43)
    check_identical(x, y, {"num_trees": 10, "max_depth": 6, "objective": "binary"}, x_test=xt)


@pytest.mark.parametrize("params", [
    {"goss": True},
    {"goss": True, "goss_top_rate": 0.3, "goss_other_rate": 0.2, "num_leaves": 23},
    {"subsample": 0.5},
    {"subsample": 0.7, "num_leaves": 31},
])
def test_goss_and_bagging_identical_trees(params):
    # Shaders.swift:1093-1221: the same rows are kept, amplified and
    # quantised, so the sampled trees and every row's prediction match
    x, y = mb.friedman(20_000, 12, 31)
    xt, _ = mb.friedman(4000, 12, 32)
    check_identical(x, y, dict({"num_trees": 25, "max_depth": 6}, **params), x_test=xt)


@pytest.mark.parametrize("params", [
    {"num_trees": 8, "max_depth": 6, "monotone_constraints": [0, 0, 0, 1, 0, -1]},
    {"num_trees": 8, "max_depth": 5, "learning_rate": 0.5, "goss": True,
     "objective": "binary"},
    {"num_trees": 8, "max_depth": 6, "num_leaves": 23},
])
def test_trees_grown_in_several_calls_equal_one_call(params):
    # A level-wise tree's deepest covers (and empty leaves) are written by the
    # next tree's first pass, or at the end of the grow call when it is the
    # last: a model grown 3 + 4 + 1 trees at a time equals one grown at once
    # and the oracle's, in every array.
    x, y = O.friedman(15_000, 6, 101)
    if params.get("objective") == "binary":
        y = (y > np.median(y)).astype(np.float32)
    cfg = {k: v for k, v in params.items() if k != "num_trees"}
    models = []
    for steps in ([8], [3, 4, 1]):
        tr = mb.Trainer(cfg, x, y, feature_major=True)
        try:
            for n in steps:
                tr.grow(n)
            models.append(model_io.saved_model(tr.booster()))
        finally:
            tr.close()
    assert models[0] == models[1]
    ref = oracle_fit(x, y, params)
    got = model_io.forest_from_json(models[1], ref.forest.nodes_per_tree)
    model_io.assert_same_forest(got, ref.forest, with_cats=False)


@pytest.mark.parametrize("params", [
    {"goss": True, "min_child_weight": 0.0},
    {"subsample": 0.6, "min_child_weight": 0.0, "min_split_gain": -1.0},
])
def test_sampled_trees_without_a_child_hessian_floor(params):
    # with min_child_weight = 0 a split may leave a child without kept rows,
    # so a sampled tree counts its deepest nodes with the partition rather
    # than in the prediction walk (which would apply such a child's leaf to
    # rows the sample left out): both paths must give the oracle's trees
    x, y = mb.friedman(20_000, 12, 35)
    xt, _ = mb.friedman(4000, 12, 36)
    check_identical(x, y, dict({"num_trees": 25, "max_depth": 6}, **params), x_test=xt)


def test_goss_logistic_nan_categorical_identical_trees():
    # GOSSTests.swift:108-130 runs GOSS with NaN and categorical features
    x, y = _mixed(15_000)
    yb = (y > np.median(y)).astype(np.float32)
    check_identical(x, yb, {"num_trees": 20, "max_depth": 5, "objective": "binary",
                            "goss": True, "categorical_features": [6]},
                    is_cat=[0] * 6 + [1], x_test=x[:, :2000].copy())


def _positive_labels(kind, rows, seed):
    # ObjectiveTests.swift:67-108: Poisson counts with rate exp(0.5 + 1.5 x0)
    # and zero-inflated positive labels for Tweedie (numpy-drawn here)
    rng = np.random.default_rng(seed)
    x = rng.random((5, rows), dtype=np.float32)
    if kind == "poisson":
        y = rng.poisson(np.exp(0.5 + 1.5 * x[0])).astype(np.float32)
    else:
        y = np.where(rng.random(rows) < 0.6, 0.0,
                     np.exp(1.0 + 2.0 * x[0]) * (0.5 + rng.random(rows))).astype(np.float32)
    return x, y


@pytest.mark.parametrize("params", [
    {"objective": "huber", "alpha": 1.5},
    {"objective": "huber", "alpha": 0.3, "num_leaves": 19},
    {"objective": "poisson"},
    {"objective": "poisson", "num_leaves": 23, "subsample": 0.7},
    {"objective": "tweedie", "tweedie_variance_power": 1.5},
    {"objective": "tweedie", "tweedie_variance_power": 1.2, "num_leaves": 17, "goss": True,
     "learning_rate": 0.3},
])
def test_huber_poisson_tweedie_identical_trees(params):
    # compute_gradients cases 3, 5 and 6 (Shaders.swift:116-130): the same
    # trees, raw scores and log-link predictions as the oracle
    kind = params["objective"]
    if kind == "huber":
        x, y = O.friedman(12_000, 8, 371)
        y = y.copy()
        y[np.random.default_rng(372).random(12_000) < 0.02] += 60.0
    else:
        x, y = _positive_labels(kind, 12_000, 373)
    check_identical(x, y, dict({"num_trees": 25, "max_depth": 5}, **params),
                    x_test=np.ascontiguousarray(x[:, :3000]))


@pytest.mark.parametrize("params", [
    {"feature_fraction": 0.5},
    {"feature_fraction": 0.3, "num_leaves": 21},
    {"allowed_features": [0, 1, 2, 3, 4]},
    {"allowed_features": [1, 3, 4, 6], "feature_fraction": 0.5, "num_leaves": 12},
    {"feature_fraction": 0.05, "objective": "binary"},
])
def test_feature_fraction_and_allowed_features_identical_trees(params):
    # per-tree column masks (Booster.swift:684-700, :1386-1400): the same
    # features are offered to every node, so the trees are the oracle's
    x, y = O.friedman(15_000, 10, 93)
    if params.get("objective") == "binary":
        y = (y > np.median(y)).astype(np.float32)
    h, ref = check_identical(x, y, dict({"num_trees": 30, "max_depth": 5}, **params),
                             x_test=np.ascontiguousarray(x[:, :3000]))
    if "allowed_features" in params:
        banned = [f for f in range(10) if f not in params["allowed_features"]]
        assert not np.isin(ref.forest.feature, banned).any()


def _first_trees(forest, k):
    return O.Forest(**{f.name: (None if getattr(forest, f.name) is None
                                else np.ascontiguousarray(getattr(forest, f.name)[:k]))
                       for f in dataclasses.fields(forest)})


def test_valid_eval_and_early_stopping_match_oracle():
    # Booster.swift:1650-1696: valid RMSE after every tree, stop after 5 stale
    # rounds, keep the best iteration's trees
    x, y = O.friedman(3000, 10, 61)
    xv, yv = O.friedman(3000, 10, 62)
    params = {"num_trees": 300, "max_depth": 6, "learning_rate": 0.3, "early_stopping_rounds": 5}
    h = mb.train(params, x, y, eval_set=(xv.T, yv), feature_major=True)
    best = mb.best_iteration(h)
    assert 1 <= best < 295 and mb.num_trees(h) == best
    ref = oracle_fit(x, y, {"num_trees": best + 5, "max_depth": 6, "learning_rate": 0.3})
    rmse = []
    for k in range(1, best + 6):
        p = O.predict(_first_trees(ref.forest, k), ref.base_score, ref.num_bins, xv)
        rmse.append(np.float32(np.sqrt(np.mean((p.astype(np.float64) - yv) ** 2))))
    rmse = np.array(rmse)
    assert int(np.argmin(rmse)) + 1 == best or np.isclose(rmse.min(), rmse[best - 1], rtol=1e-6)
    assert (rmse[best:] >= rmse[best - 1] * (1 - 1e-6)).all()      # the 5 stale rounds
    got = model_io.forest_from_json(model_io.saved_model(h), ref.forest.nodes_per_tree)
    model_io.assert_same_forest(got, _first_trees(ref.forest, best), with_cats=False)


# --------------------------------------------------------------------------
# L1 / quantile objectives: leaf renewal
# --------------------------------------------------------------------------

def _outlier_friedman(rows, cols, seed):
    x, y = O.friedman(rows, cols, seed)
    rng = np.random.default_rng(seed)
    y = y.copy()
    y[rng.random(rows) < 0.02] += 100.0
    return x, y


@pytest.mark.parametrize("params", [
    {"num_trees": 30, "max_depth": 6, "objective": "mae"},
    {"num_trees": 30, "max_depth": 5, "objective": "quantile", "alpha": 0.9},
    {"num_trees": 25, "max_depth": 6, "num_leaves": 20, "objective": "quantile", "alpha": 0.2},
    {"num_trees": 25, "max_depth": 7, "num_leaves": 40, "objective": "mae"},
    {"num_trees": 25, "max_depth": 5, "objective": "mae", "goss": True, "learning_rate": 0.3},
    {"num_trees": 20, "max_depth": 6, "objective": "quantile", "alpha": 0.7,
     "monotone_constraints": [1, 0, 0, 0, 0, 0, -1, 0]},
])
def test_leaf_renewal_identical_trees(params):
    # Booster.swift:634-639, :1241-1290, :1596-1615
    x, y = _outlier_friedman(30_000, 8, 91)
    xt, _ = O.friedman(5000, 8, 92)
    check_identical(x, y, params, x_test=xt)


def test_leaf_renewal_strided_sample_identical():
    # more than 2 * 262144 rows: renewal samples every other row, and the base
    # score every third label
    x, y = _outlier_friedman(600_000, 5, 93)
    check_identical(x, y, {"num_trees": 4, "max_depth": 6, "objective": "quantile",
                           "alpha": 0.6})


def test_leaf_renewal_nan_categorical_identical():
    x, y, cats = D.c3_mixed(40_000, 7)
    is_cat = [0] * 80 + [1] * 20
    check_identical(x, y, {"num_trees": 10, "max_depth": 6, "objective": "mae",
                           "categorical_features": cats}, is_cat=is_cat)


# --------------------------------------------------------------------------
# multiclass (softmax, K trees per round)
# --------------------------------------------------------------------------

def _quadrant_classes(rows, seed, cols=5):
    rng = np.random.default_rng(seed)
    x = rng.uniform(0, 1, size=(cols, rows)).astype(np.float32)
    a = (x[0] + 0.15 * rng.standard_normal(rows) > 0.5).astype(int)
    b = (x[1] + 0.15 * rng.standard_normal(rows) > 0.5).astype(int) * 2
    return x, (a + b).astype(np.float32)


def check_identical_mc(x_fm, y, params, is_cat=None, x_test=None):
    K = params["num_class"]
    h, obj = gpu_fit(x_fm, y, params)
    ref = oracle_fit(x_fm, y, params, is_cat)
    assert mb.num_classes(h) == K and obj["numClasses"] == K
    assert np.array_equal(np.array(obj["baseScores"], np.float32),
                          np.array(ref.base_scores, np.float32))
    got = model_io.forest_from_json(obj, ref.forest.nodes_per_tree)
    has_cats = is_cat is not None and any(is_cat)
    model_io.assert_same_forest(got, ref.forest, with_cats=has_cats)
    # running train preds [K][rows] == the forest walk, bit for bit
    assert np.array_equal(mb.predict(h, x_fm, feature_major=True), ref.preds.T)
    if x_test is not None:
        gp = mb.predict(h, x_test, feature_major=True)
        assert gp.shape == (x_test.shape[1], K)
        assert np.array_equal(gp, O.predict_mc(ref.forest, ref.base_scores, ref.num_bins, x_test))
    return h, ref


@pytest.mark.parametrize("params", [
    {"num_trees": 15, "max_depth": 5, "objective": "multiclass", "num_class": 4},
    {"num_trees": 10, "max_depth": 6, "objective": "multiclass", "num_class": 3,
     "learning_rate": 0.3, "lambda": 2.0},
    {"num_trees": 10, "max_depth": 7, "num_leaves": 15, "objective": "multiclass",
     "num_class": 4},
    {"num_trees": 10, "max_depth": 5, "objective": "multiclass", "num_class": 4,
     "subsample": 0.7},
])
def test_multiclass_identical_trees(params):
    # ObjectiveTests.swift:519-557; LeafWiseTests.swift:105-125
    x, y = _quadrant_classes(20_000, 121)
    if params["num_class"] == 3:
        y = np.minimum(2, (x[0] * 3).astype(int)).astype(np.float32)
    xt, _ = _quadrant_classes(4000, 122)
    h, ref = check_identical_mc(x, y, params, x_test=xt)
    assert mb.num_trees(h) == params["num_trees"] * params["num_class"]


def test_multiclass_nan_categorical_identical_trees():
    rows = 20_000
    x, y = _quadrant_classes(rows, 7)
    x[3, ::9] = np.nan
    x[4] = np.floor(x[4] * 12)
    y = np.where(x[4] == 5, 3, y).astype(np.float32)
    check_identical_mc(x, y, {"num_trees": 8, "max_depth": 6, "objective": "multiclass",
                              "num_class": 4, "categorical_features": [4]},
                       is_cat=[0, 0, 0, 0, 1], x_test=x[:, :3000].copy())


def test_multiclass_shap_and_save_load(tmp_path):
    # ObjectiveTests.swift:480-513: per-class blocks sum to the class score;
    # GPU contributions equal the oracle's per class; save/load is bitwise
    rows, cols, K = 800, 4, 3
    rng = np.random.default_rng(131)
    x = rng.uniform(0, 1, size=(cols, rows)).astype(np.float32)
    y = np.minimum(2, (x[0] * 3).astype(int)).astype(np.float32)
    params = {"num_trees": 25, "max_depth": 4, "objective": "multiclass", "num_class": K}
    h = mb.train(params, x, y, feature_major=True)
    ref = oracle_fit(x, y, params)
    c = mb.predict_contrib(h, x, feature_major=True).reshape(rows, K, cols + 1)
    raw = mb.predict(h, x, feature_major=True)
    assert np.abs(c.sum(axis=2) - raw).max() < 1e-4
    want = O.treeshap_mc(ref.forest, ref.base_scores, ref.num_bins, x).reshape(rows, K, cols + 1)
    assert np.allclose(c, want, rtol=1e-5, atol=1e-6)
    mb.save(h, tmp_path / "mc.json")
    h2 = mb.load(tmp_path / "mc.json")
    assert np.array_equal(mb.predict(h2, x, feature_major=True), raw)


def test_multiclass_early_stopping_keeps_whole_rounds():
    # Booster.swift:1650-1696: multi_logloss once per round of K trees; the
    # best round's K * best trees are kept
    K = 4
    x, y = _quadrant_classes(6000, 31)
    xv, yv = _quadrant_classes(3000, 32)
    params = {"num_trees": 300, "max_depth": 4, "learning_rate": 0.5, "objective": "multiclass",
              "num_class": K}
    h = mb.train(dict(params, early_stopping_rounds=4), x, y, eval_set=(xv.T, yv),
                 feature_major=True)
    best = mb.best_iteration(h)
    assert 1 <= best < 296 and mb.num_trees(h) == best * K
    ref = oracle_fit(x, y, dict(params, num_trees=best + 4))

    def mlogloss(p):
        z = p.astype(np.float64)
        m = z.max(axis=1)
        lse = np.log(np.exp(z - m[:, None]).sum(axis=1)) + m
        return float(np.mean(lse - z[np.arange(len(yv)), yv.astype(int)]))

    losses = np.array([mlogloss(O.predict_mc(_first_trees(ref.forest, r * K), ref.base_scores,
                                             ref.num_bins, xv)) for r in range(1, best + 5)],
                      np.float32)
    assert int(np.argmin(losses)) + 1 == best or np.isclose(losses.min(), losses[best - 1],
                                                             rtol=1e-6)
    assert (losses[best:] >= losses[best - 1] * (1 - 1e-6)).all()    # the 4 stale rounds
    got = model_io.forest_from_json(model_io.saved_model(h), ref.forest.nodes_per_tree)
    model_io.assert_same_forest(got, _first_trees(ref.forest, best * K), with_cats=False)


# --------------------------------------------------------------------------
# warm start (init_model)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("params,rm", [
    ({"max_depth": 5}, False),
    ({"max_depth": 6, "num_leaves": 20, "objective": "binary"}, True),
    ({"max_depth": 4, "objective": "multiclass", "num_class": 3}, False),
])
def test_warm_start_continues_one_shot_training(tmp_path, params, rm):
    # ObjectiveTests.swift:374-393.  The init model's raw scores equal the
    # running predictions after its trees, so 20 + 20 trees are the one-shot
    # run's 40 trees.
    rows = 20_000
    x, y = O.friedman(rows, 8, 105)
    if params.get("objective") == "binary":
        y = (y > np.median(y)).astype(np.float32)
    if params.get("objective") == "multiclass":
        y = np.minimum(2, (x[0] * 3).astype(int)).astype(np.float32)
    first = mb.train(dict(params, num_trees=20), x, y, feature_major=True)
    mb.save(first, tmp_path / "first.json")
    xin = np.ascontiguousarray(x.T) if rm else x
    second = mb.train(dict(params, num_trees=20, init_model=str(tmp_path / "first.json")), xin,
                      y, feature_major=not rm)
    full = mb.train(dict(params, num_trees=40), x, y, feature_major=True)
    K = params.get("num_class", 1)
    assert mb.num_trees(second) == 40 * K
    a, b = model_io.saved_model(second), model_io.saved_model(full)
    nodes = (1 << (params["max_depth"] + 1)) - 1
    model_io.assert_same_forest(model_io.forest_from_json(a, nodes),
                                model_io.forest_from_json(b, nodes), with_cats=False)
    assert a["baseScore"] == b["baseScore"] and a["baseScores"] == b["baseScores"]
    xt, _ = O.friedman(3000, 8, 106)
    assert np.array_equal(mb.predict(second, xt, feature_major=True),
                          mb.predict(full, xt, feature_major=True))


def test_warm_start_with_validation_set(tmp_path):
    x, y = O.friedman(15_000, 8, 107)
    xv, yv = O.friedman(4000, 8, 108)
    first = mb.train({"num_trees": 15, "max_depth": 5}, x, y, feature_major=True)
    mb.save(first, tmp_path / "f.json")
    p = {"num_trees": 200, "max_depth": 5, "learning_rate": 0.3, "early_stopping_rounds": 5,
         "init_model": str(tmp_path / "f.json")}
    second = mb.train(p, x, y, eval_set=(xv.T, yv), feature_major=True)
    best = mb.best_iteration(second)
    assert mb.num_trees(second) == 15 + best
    ref = oracle_fit(x, y, {"num_trees": 15 + best + 5, "max_depth": 5})
    got = model_io.forest_from_json(model_io.saved_model(second), ref.forest.nodes_per_tree)
    first_f = model_io.forest_from_json(model_io.saved_model(first), ref.forest.nodes_per_tree)
    model_io.assert_same_forest(first_f, _first_trees(ref.forest, 15), with_cats=False)
    assert got.num_trees == 15 + best


# --------------------------------------------------------------------------
# Boruta feature selection (macboost_select_features)
# --------------------------------------------------------------------------

def _signal_plus_noise(rows, signal=5, noise=5, seed=311):
    x, y = O.friedman(rows, signal, seed)
    rng = np.random.default_rng(seed + 1)
    return np.vstack([x, rng.uniform(0, 1, (noise, rows)).astype(np.float32)]), y


@pytest.mark.parametrize("params,seed", [({"num_trees": 30, "max_depth": 6}, 0),
                                         ({"num_trees": 20, "max_depth": 5, "num_bins": 64}, 77)])
def test_select_features_matches_oracle(params, seed):
    # FeatureSelection.swift:45-190: the same shadows, the same probe models,
    # so the same votes, decisions and gain ratios
    x, y = _signal_plus_noise(6000)
    hits, dec, ratio = mb.select_features(params, x, y, rounds=8, seed=seed, feature_major=True)
    kw = dict(params)
    nb = kw.pop("num_bins", 256)
    nt = kw.pop("num_trees")
    oh, od, orat = O.select_features(x, y, rounds=8, seed=seed, num_bins=nb, num_trees=nt, **kw)
    assert np.array_equal(hits, oh) and np.array_equal(dec, od)
    assert np.array_equal(ratio, orat)
    assert (hits[:5] >= 7).all()                       # the signal beats every shadow


def test_select_features_nan_categorical_and_rows_not_a_power_of_two():
    # SelectionTests.swift:80-100: shadows of a categorical column stay categorical
    rows = 5001
    x, y = O.friedman(rows, 5, 351)
    rng = np.random.default_rng(352)
    x = x.copy()
    x[2, rng.random(rows) < 0.2] = np.nan
    good = rng.integers(0, 6, rows).astype(np.float32)
    junk = rng.integers(0, 6, rows).astype(np.float32)
    y = (y + np.where(good == 3, 4.0, 0.0)).astype(np.float32)
    x = np.vstack([x, good[None], junk[None]])
    params = {"num_trees": 25, "max_depth": 5, "categorical_features": [5, 6]}
    hits, dec, ratio = mb.select_features(params, x, y, rounds=6, trees=20, seed=5,
                                          feature_major=True)
    is_cat = np.array([0, 0, 0, 0, 0, 1, 1], np.uint8)
    oh, od, orat = O.select_features(x, y, rounds=6, trees=20, seed=5, num_trees=25,
                                     max_depth=5, is_cat=is_cat)
    assert np.array_equal(hits, oh) and np.array_equal(dec, od) and np.array_equal(ratio, orat)
    assert hits[5] == 6 and hits[6] < 6


# --------------------------------------------------------------------------
# leaf-wise (best-first) growth
# --------------------------------------------------------------------------

@pytest.mark.parametrize("num_leaves,depth", [(31, 6), (2, 6), (64, 6), (17, 12)])
def test_leafwise_identical_trees(num_leaves, depth):
    # num_leaves = 2^depth reaches every level (the level-wise shape); 2 gives stumps
    x, y = mb.friedman(20_000, 30, 77)
    xt, _ = mb.friedman(5_000, 30, 77 + 999)
    check_identical(x, y, {"num_trees": 20, "max_depth": depth, "num_leaves": num_leaves,
                           "num_bins": 128}, x_test=xt)


@pytest.mark.parametrize("num_leaves", [5, 11, 23])
def test_leafwise_equal_gains_identical(num_leaves):
    # Two mirrored halves: the same rows, a flag feature that is 0 in one half
    # and 1 in the other, and integer labels reflected about their mean, so
    # every L2 gradient of one half is exactly the negation of its twin's.
    # The root splits on the flag and every node of one subtree has a twin of
    # exactly equal gain: the best-first picks break ties by open-list order
    # (5 and 11 leaves end with one more split on the left side than the right).
    rng = np.random.default_rng(2024)
    n, c = 3000, 40
    xa = rng.random((5, n), dtype=np.float32)
    ya = np.round(12 * xa[0] + 6 * xa[1] ** 2 + rng.integers(0, 3, n)).astype(np.float32)
    x = np.concatenate([np.concatenate([xa, xa], axis=1),
                        np.concatenate([np.zeros(n), np.ones(n)])[None].astype(np.float32)])
    y = np.concatenate([ya, 2 * c - ya]).astype(np.float32)
    check_identical(np.ascontiguousarray(x), y, {"num_trees": 6, "max_depth": 6,
                                                 "num_leaves": num_leaves, "num_bins": 64})


def test_leafwise_nan_categorical_monotone_identical():
    x, y = _mixed(12_000)
    params = {"num_trees": 20, "max_depth": 6, "num_leaves": 24, "categorical_features": [6],
              "monotone_constraints": [0, 0, 0, 1, 0, 0, 0]}
    h, ref = check_identical(x, y, params, is_cat=[0] * 6 + [1], x_test=x[:, :3000].copy())
    assert (ref.forest.flags & O.FLAG_CATEGORICAL).any()


def _leaves(tree):
    feat = tree["feature"]
    reach, n_leaves, stack = set(), 0, [0]
    while stack:
        n = stack.pop()
        reach.add(n)
        if feat[n] >= 0:
            stack += [2 * n + 1, 2 * n + 2]
        else:
            n_leaves += 1
    return n_leaves


def test_leafwise_budget_and_stumps():
    # LeafWiseTests.swift:68-103 (leaf budget) and :219-240 (numLeaves=2 stumps)
    x, y = O.friedman(8000, 8, 5)
    _, obj = gpu_fit(x, y, {"num_trees": 6, "max_depth": 6, "num_leaves": 7})
    assert all(_leaves(t) <= 7 for t in obj["trees"])
    assert max(_leaves(t) for t in obj["trees"]) == 7
    _, obj = gpu_fit(x, y, {"num_trees": 6, "max_depth": 6, "num_leaves": 2})
    for t in obj["trees"]:
        assert t["feature"][0] >= 0 and t["feature"][1] == -1 and t["feature"][2] == -1


# --------------------------------------------------------------------------
# TreeSHAP
# --------------------------------------------------------------------------

def _mixed(rows, seed_a=211, seed_b=212, nan_frac=0.15):
    x, y = O.friedman(rows, 6, seed_a)
    rng = O.SplitMix(seed_b)
    nan = O.SplitMix(seed_b + 1).uniforms(rows) < nan_frac
    x[1, nan] = np.nan
    cat = np.array([rng.next() % 5 for _ in range(rows)], np.float32)
    x = np.vstack([x, cat[None, :]])
    y = (y + np.where(cat == 2, 3.0, 0.0)).astype(np.float32)
    return x, y


@pytest.mark.parametrize("depth", [3, 6, 8, 12])
def test_treeshap_matches_oracle(depth):
    # ObjectiveTests.swift:440-478 (tolerance tightened from 5e-3 abs); the
    # depths cover every per-lane array size of the path-parallel kernel
    x, y = _mixed(3000)
    h, obj = gpu_fit(x, y, {"num_trees": 40 if depth <= 8 else 8, "max_depth": depth,
                            "categorical_features": [6]})
    c = mb.predict_contrib(h, x, feature_major=True)
    forest = model_io.forest_from_json(obj)
    want = O.treeshap(forest, obj["baseScore"], obj["numBins"], x)
    assert np.allclose(c, want, rtol=1e-5, atol=1e-6)
    # reproducible run to run (each row's phi is summed by one wavefront)
    assert np.array_equal(c, mb.predict_contrib(h, x, feature_major=True))
    raw = mb.predict(h, x, feature_major=True)
    assert np.max(np.abs(c.astype(np.float64).sum(axis=1) - raw)) < 1e-4


def test_treeshap_wide_data_matches_oracle():
    # more columns than the path-parallel kernel keeps in LDS: the lane-per-row
    # kernel with its global phi scratch
    rows, cols = 1200, 4100
    x, y = O.friedman(rows, cols, 37)
    h, obj = gpu_fit(x, y, {"num_trees": 6, "max_depth": 4})
    c = mb.predict_contrib(h, x, feature_major=True)
    assert c.shape == (rows, cols + 1)
    want = O.treeshap(model_io.forest_from_json(obj), obj["baseScore"], obj["numBins"], x)
    assert np.allclose(c, want, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------
# Row checks and the base score's sums on the device (k_label_stats)
# --------------------------------------------------------------------------

def test_device_row_checks_messages():
    # the first offending row over every block, with the reference's message
    # (Booster.swift:1724-1765); labels before weights before categoricals
    rows = 200_000
    x = np.random.default_rng(1).random((3, rows), dtype=np.float32)
    y = np.zeros(rows, np.float32)
    bad = y.copy()
    bad[[150_001, 170_000]] = np.nan
    with pytest.raises(mb.MacBoostError, match=r"label at row 150001 is nan; labels must be finite"):
        mb.train({"num_trees": 1}, x, bad, feature_major=True)
    yb = (np.arange(rows) % 2).astype(np.float32)
    yb[65_536] = 2.0
    with pytest.raises(mb.MacBoostError,
                       match=r"label at row 65536 is 2.0; binary objective requires labels in \{0, 1\}"):
        mb.train({"num_trees": 1, "objective": "binary"}, x, yb, feature_major=True)
    w = np.ones(rows, np.float32)
    w[[99_999, 131_072]] = -1.0
    with pytest.raises(mb.MacBoostError, match=r"weight at row 99999 is -1.0; weights must be finite"):
        mb.train({"num_trees": 1}, x, y, feature_major=True, sample_weight=w)
    # a bad label wins over a bad weight and over a bad categorical value
    xc = x.copy()
    xc[0, 5] = 999.0
    with pytest.raises(mb.MacBoostError, match=r"label at row 150001 is nan"):
        mb.train({"num_trees": 1, "categorical_features": [0]}, xc, bad, feature_major=True,
                 sample_weight=w)


@pytest.mark.parametrize("case", ["cancel", "l2", "logistic_w", "poisson"])
def test_device_base_score_matches_oracle(case):
    rng = np.random.default_rng(11)
    rows = 130 if case == "cancel" else 200_003
    x = rng.random((2, rows), dtype=np.float32)
    w = None
    params = {"num_trees": 1, "max_depth": 2}
    if case == "cancel":
        y = np.ones(rows, np.float32)
        y[0], y[64] = 1e17, -1e17
        obj = O.OBJ_L2
    elif case == "l2":
        y = (rng.standard_normal(rows) * 1e3 + 0.1).astype(np.float32)
        obj = O.OBJ_L2
    elif case == "logistic_w":
        y = (rng.random(rows) < 0.3).astype(np.float32)
        w = rng.random(rows).astype(np.float32)
        params.update(objective="binary", scale_pos_weight=2.5)
        obj = O.OBJ_LOGISTIC
    else:
        y = rng.poisson(3.0, rows).astype(np.float32)
        params.update(objective="poisson")
        obj = O.OBJ_POISSON
    h = mb.train(params, x, y, feature_major=True, sample_weight=w)
    got = np.float32(model_io.saved_model(h)["baseScore"])
    spw = 2.5 if case == "logistic_w" else 1.0
    assert got == np.float32(O.base_score(y, w, obj, spw))
    if case == "cancel":
        assert got == np.float32(128 / 130)
