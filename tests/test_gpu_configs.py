"""GPU parity at the benchmark configurations' own shapes, through the C ABI.

* 10M x 100 Friedman #1, 256 bins: leaf-wise with 63 leaves (2 trees) and
  level-wise depth 6 (1 tree), every model array equal to the oracle's.  A
  63-leaf depth-6 tree grows in depth rounds on the level-wise partition; the
  level-wise tree also reads the planar root copy.
* 5M x 20 Friedman #1, leaf-wise with 63 leaves and max_depth 10 (2 trees):
  trees deeper than 8 grow one leaf per step, and the root segment (5M
  entries) is larger than the per-step partition grid (512 blocks x 8,192
  entries), so its grid-stride loop and the plan run by the block that
  reserves a segment's last entries are compared with the oracle.
* HIGGS-like 10.5M x 28 logistic (the training 10M rows): 2 plain trees, and
  4 GOSS (0.2, 0.1) trees at learning rate 0.5, whose trees 2 and 3 sample
  their rows past the ceil(1/lr) = 2 warm-up trees.
* 100 leaf-wise trees on the same data: 500k held-out rows predicted bit for
  bit against the oracle's predictCPU restatement, and TreeSHAP of 200k rows
  within 1e-5 relative of the oracle on 2,000 of them (every 100th), with all
  200k rows summing to their predictions.
* HIGGS-like 200k x 28 logistic with GOSS (0.2, 0.1): 20 trees, past the
  ceil(1/lr) = 10 warm-up trees.
* 1M x 100 with 20 categorical columns and 20% NaN, with the 200k-row
  validation set scored after every tree: the per-iteration metric and the
  best iteration equal the oracle's.

The oracle runs on every host core (its results do not depend on the thread
count); each case prints what it runs before it starts.
"""
import sys

import numpy as np
import pytest

import datasets as D
import macboost_amd as mb
import model_io
import oracle_lib as O
from test_gpu_parity import _first_trees, check_identical, oracle_fit

pytestmark = pytest.mark.gpu

ROWS, COLS = 10_000_000, 100


def say(msg):
    print(f"[configs] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def friedman10m():
    O.set_threads(0)
    say("generating Friedman #1 10M x 100 (seed 42)")
    x, y = mb.friedman(ROWS, COLS, 42)
    say("oracle edges + bins")
    edges = O.compute_edges(x, 256)
    bins = O.bin_matrix(x, edges, 256)
    return x, y, edges, bins


def _compare(x, y, edges, bins, params, **okw):
    h = mb.train(params, x, y, feature_major=True)
    obj = model_io.saved_model(h)
    ref = O.fit(bins, y, edges=edges, num_bins=256, num_trees=params["num_trees"],
                max_depth=params.get("max_depth", 6), num_leaves=params.get("num_leaves", 0),
                **okw)
    got = model_io.forest_from_json(obj, ref.forest.nodes_per_tree)
    assert np.float32(obj["baseScore"]) == np.float32(ref.base_score)
    model_io.assert_same_forest(got, ref.forest, with_cats=False)
    assert np.array_equal(mb.predict(h, x, feature_major=True), ref.preds)
    return h, ref


def test_c5_leafwise_63_leaves_identical_trees(friedman10m):
    say("10M x 100 leaf-wise 63 leaves, 2 trees: GPU vs oracle")
    x, y, edges, bins = friedman10m
    _, ref = _compare(x, y, edges, bins, {"num_trees": 2, "max_depth": 6, "num_leaves": 63,
                                          "num_bins": 256})
    # the full budget was used: 62 splits per tree
    assert ((ref.forest.feature >= 0).sum(axis=1) == 62).all()


def test_metric_run_levelwise_depth6_identical_tree(friedman10m):
    say("10M x 100 level-wise depth 6, 1 tree: GPU vs oracle")
    x, y, edges, bins = friedman10m
    _, ref = _compare(x, y, edges, bins, {"num_trees": 1, "max_depth": 6, "num_bins": 256})
    assert (ref.forest.feature[0, :63] >= 0).all()       # a full depth-6 tree


def test_c5_predict_500k_bitexact_and_treeshap(friedman10m):
    x, y, _, _ = friedman10m
    say("10M x 100 leaf-wise 63 leaves, 100 trees on the GPU")
    h = mb.train({"num_trees": 100, "max_depth": 6, "num_leaves": 63, "num_bins": 256},
                 x, y, feature_major=True)
    obj = model_io.saved_model(h)
    forest = model_io.forest_from_json(obj)
    assert forest.num_trees == 100
    base, nb = obj["baseScore"], obj["numBins"]
    xp, _ = mb.friedman(500_000, COLS, 42 + 999)
    say("predict 500k rows x 100 trees: GPU vs oracle")
    got = mb.predict(h, xp, feature_major=True)
    assert np.array_equal(got, O.predict(forest, base, nb, xp))
    xs = np.ascontiguousarray(xp[:, :200_000])
    say("TreeSHAP 200k rows x 100 trees on the GPU, 2,000 rows vs oracle")
    c = mb.predict_contrib(h, xs, feature_major=True)
    assert c.shape == (200_000, COLS + 1)
    pick = np.arange(0, 200_000, 100)
    want = O.treeshap(forest, base, nb, np.ascontiguousarray(xs[:, pick]))
    assert np.allclose(c[pick], want, rtol=1e-5, atol=1e-6)
    # every row's contributions sum to its raw prediction
    s = c.astype(np.float64).sum(axis=1)
    assert np.max(np.abs(s - got[:200_000])) < 1e-3


def test_leafwise_per_step_depth10_large_root_segment():
    # LeafWiseTests.swift:205-217 grows best-first trees to a depth limit; past
    # depth 8 this library grows them one leaf per step.
    rows, cols = 5_000_000, 20
    assert rows > 512 * 8192
    O.set_threads(0)
    say(f"{rows} x {cols} leaf-wise 63 leaves, max_depth 10, 2 trees: GPU vs oracle")
    x, y = mb.friedman(rows, cols, 7)
    edges = O.compute_edges(x, 256)
    bins = O.bin_matrix(x, edges, 256)
    _, ref = _compare(x, y, edges, bins, {"num_trees": 2, "max_depth": 10, "num_leaves": 63,
                                          "num_bins": 256})
    assert ((ref.forest.feature >= 0).sum(axis=1) == 62).all()
    # best-first went past depth 6 somewhere (a node index beyond a depth-6 heap)
    deep = [np.nonzero(ref.forest.feature[t] >= 0)[0].max() for t in range(2)]
    assert max(deep) >= 127


@pytest.fixture(scope="module")
def higgs10m():
    say("generating HIGGS-like 10.5M x 28 (seed 42), training rows 10M")
    x, y = D.c4_higgs_like(10_500_000, 42)
    return np.ascontiguousarray(x[:, :10_000_000]), np.ascontiguousarray(y[:10_000_000])


def test_c4_10m_plain_identical_trees(higgs10m):
    # README.md:62: HIGGS 10.5M x 28, binary logistic, 256 bins, depth 6
    x, y = higgs10m
    say("HIGGS-like 10M x 28 logistic, 2 trees: GPU vs oracle")
    O.set_threads(0)
    check_identical(x, y, {"num_trees": 2, "max_depth": 6, "num_bins": 256,
                           "objective": "binary"})


def test_c4_10m_goss_identical_trees(higgs10m):
    # GOSSTests.swift:85-110; README.md:63: GOSS (0.2, 0.1). At lr 0.5 the
    # warm-up is ceil(1/0.5) = 2 trees, so trees 2 and 3 sample their rows.
    x, y = higgs10m
    say("HIGGS-like 10M x 28 logistic + GOSS(0.2, 0.1), lr 0.5, 4 trees: GPU vs oracle")
    O.set_threads(0)
    check_identical(x, y, {"num_trees": 4, "max_depth": 6, "num_bins": 256,
                           "objective": "binary", "learning_rate": 0.5, "goss": True,
                           "goss_top_rate": 0.2, "goss_other_rate": 0.1})


def test_c4_goss_identical_trees():
    # HIGGS-like logistic with GOSS (0.2, 0.1): trees 10..19 sample their rows
    say("HIGGS-like 200k x 28 logistic + GOSS(0.2, 0.1), 20 trees: GPU vs oracle")
    O.set_threads(0)
    x, y = D.c4_higgs_like(200_000, 42)
    xt, _ = D.c4_higgs_like(50_000, 43)
    params = {"num_trees": 20, "max_depth": 6, "num_bins": 256, "objective": "binary",
              "goss": True, "goss_top_rate": 0.2, "goss_other_rate": 0.1}
    check_identical(x, y, params, x_test=xt)
    assert O.sample_rows(np.ones(4, np.float32), np.ones(4, np.float32), 1.0, 10,
                         goss=True) is not None                   # tree 10 samples


def _rmse_sequential(pred, y):
    # the trainer's metric: a sequential double sum of squares, sqrt, f32
    d = pred.astype(np.float64) - y.astype(np.float64)
    return np.float32(np.sqrt(np.cumsum(d * d)[-1] / len(y)))


def test_c3_validation_metric_every_tree():
    say("1M x 100, 20 categorical, 20% NaN, 200k validation rows, 20 trees: GPU vs oracle")
    O.set_threads(0)
    x, y, cats = D.c3_mixed(1_000_000, 42)
    xv, yv, _ = D.c3_mixed(200_000, 42 + 999)
    params = {"num_trees": 20, "max_depth": 6, "num_bins": 256, "categorical_features": cats}
    h = mb.train(params, x, y, eval_set=(xv.T, yv), feature_major=True)
    obj = model_io.saved_model(h)
    is_cat = [0] * 80 + [1] * 20
    ref = oracle_fit(x, y, params, is_cat)
    got = model_io.forest_from_json(obj, ref.forest.nodes_per_tree)
    model_io.assert_same_forest(got, ref.forest, with_cats=True)
    hist = mb.eval_history(h)
    assert hist.shape == (20,)
    want = []
    for k in range(1, 21):
        sub = _first_trees(ref.forest, k)
        want.append(_rmse_sequential(O.predict(sub, ref.base_score, 256, xv), yv))
    assert np.array_equal(hist, np.array(want, np.float32))
    best = int(np.argmin(np.array(want))) + 1             # first minimum (strict <)
    assert mb.best_iteration(h) == best
