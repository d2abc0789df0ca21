"""GPU parity over randomised trainer settings.

Each case draws a small problem and a parameter set from its own seed:
objective (L2, logistic, L1, quantile, Huber, Poisson, Tweedie), depth 1-9,
level-wise or leaf-wise, 4-256 bins, categorical and NaN-holed columns,
min_split_gain / lambda / min_child_weight, GOSS or bagging, feature
fraction and monotone constraints; the GPU model must equal the oracle's in
every array, and its predictions on the training rows and on held-out rows
(unseen categories, NaN) bit for bit (check_identical).  The
same draws with sample weights (zeros included), multiclass draws, and the
TreeSHAP values of drawn models (within 1e-5 relative of the oracle's).
"""
import numpy as np
import pytest

import macboost_amd as mb
import model_io
import oracle_lib as O
from test_gpu_parity import check_identical, check_identical_mc, gpu_fit

pytestmark = pytest.mark.gpu

OBJECTIVES = ["regression", "binary", "mae", "quantile", "huber", "poisson", "tweedie"]


def draw_case(seed):
    rng = np.random.default_rng(seed)
    f = int(rng.integers(1, 61))
    n = int(rng.integers(1, max(2, min(150_000, 3_000_000 // f))))
    depth = int(rng.integers(1, 10))
    nb = int(rng.choice([4, 16, 32, 64, 128, 256]))
    obj = OBJECTIVES[int(rng.integers(0, len(OBJECTIVES)))]
    x = rng.random((f, n), dtype=np.float32)
    x[rng.random((f, n)) < rng.random() * 0.3] = np.nan
    ncat = int(rng.integers(0, min(3, f) + 1))
    cats = sorted(rng.choice(f, ncat, replace=False).tolist()) if ncat else []
    for c in cats:
        x[c] = rng.integers(0, int(rng.integers(2, max(3, min(40, nb - 1)))), n).astype(np.float32)
    base = np.nan_to_num(x[0], nan=0.5) * 3 + (np.nan_to_num(x[-1]) if f > 1 else 0)
    if obj == "binary":
        y = (base + rng.standard_normal(n) > base.mean()).astype(np.float32)
    elif obj in ("poisson", "tweedie"):
        y = rng.poisson(np.exp(base / 3)).astype(np.float32)
    else:
        y = (base + rng.standard_normal(n)).astype(np.float32)
    p = {"num_trees": int(rng.integers(1, 6)), "max_depth": depth, "num_bins": nb,
         "objective": obj, "learning_rate": float(rng.choice([0.05, 0.1, 0.3, 0.7]))}
    if cats:
        p["categorical_features"] = cats
    if obj == "quantile":
        p["alpha"] = float(rng.choice([0.2, 0.5, 0.9]))
    if obj == "huber":
        p["alpha"] = 1.0
    if obj == "tweedie":
        p["tweedie_variance_power"] = 1.5
    if rng.random() < 0.3:
        p["min_split_gain"] = float(rng.random())
    if rng.random() < 0.3:
        p["lambda"] = float(rng.choice([0.0, 0.5, 3.0]))
    if rng.random() < 0.3:
        p["min_child_weight"] = float(rng.choice([0.1, 1.0, 5.0]))
    if rng.random() < 0.3 and depth >= 2:
        p["num_leaves"] = int(rng.integers(2, min(2 ** depth, 64) + 1))
    r = rng.random()
    if r < 0.15:
        p.update({"goss": True, "goss_top_rate": 0.2, "goss_other_rate": 0.1})
    elif r < 0.3:
        p["subsample"] = float(rng.choice([0.5, 0.8]))
    if rng.random() < 0.2:
        p["feature_fraction"] = float(rng.choice([0.5, 0.8]))
    if rng.random() < 0.2:
        num = [i for i in range(f) if i not in cats]
        if num:
            p["monotone_constraints"] = [int(rng.choice([-1, 0, 1])) if i in num else 0
                                         for i in range(f)]
    return np.ascontiguousarray(x), y, p, [1 if i in cats else 0 for i in range(f)]


def held_out(x, is_cat, seed):
    # 500 held-out rows: values past the training range, NaN holes, and for
    # categorical columns unseen, negative and non-integer codes
    rng = np.random.default_rng(seed)
    f = x.shape[0]
    xt = (rng.random((f, 500)) * 1.4 - 0.2).astype(np.float32)
    xt[rng.random((f, 500)) < 0.2] = np.nan
    for c in range(f):
        if is_cat[c]:
            xt[c] = (rng.integers(-2, 300, 500) + rng.choice([0.0, 0.3, 0.5], 500)).astype(np.float32)
    return np.ascontiguousarray(xt)


@pytest.mark.parametrize("case", range(80))
def test_random_settings_identical(case):
    x, y, params, is_cat = draw_case(20261202 + case)
    check_identical(x, y, params, is_cat=is_cat, x_test=held_out(x, is_cat, case))


@pytest.mark.parametrize("case", range(30))
def test_random_weighted_settings_identical(case):
    x, y, params, is_cat = draw_case(20261302 + case)
    rng = np.random.default_rng(case)
    w = (rng.random(y.shape[0]) * 2.0).astype(np.float32)
    w[rng.random(y.shape[0]) < 0.1] = 0.0             # rows that count for nothing
    check_identical(x, y, params, is_cat=is_cat, w=w)


@pytest.mark.parametrize("case", range(15))
def test_random_multiclass_settings_identical(case):
    x, _, params, is_cat = draw_case(20261402 + case)
    rng = np.random.default_rng(1000 + case)
    k = int(rng.integers(3, 6))
    base = np.nan_to_num(x[0], nan=0.5) + 0.3 * rng.standard_normal(x.shape[1])
    y = np.clip((base * k).astype(np.int64), 0, k - 1).astype(np.float32)
    # GOSS with multiclass is rejected, as the reference rejects it
    params = {key: v for key, v in params.items()
              if key not in ("objective", "alpha", "tweedie_variance_power", "goss",
                             "goss_top_rate", "goss_other_rate")}
    params.update(objective="multiclass", num_class=k)
    check_identical_mc(x, y, params, is_cat=is_cat)


@pytest.mark.parametrize("case", range(20))
def test_random_settings_treeshap(case):
    x, y, params, _ = draw_case(20261502 + case)
    rows = min(x.shape[1], 1500)
    h, obj = gpu_fit(x, y, params)
    xs = np.ascontiguousarray(x[:, :rows])
    got = mb.predict_contrib(h, xs, feature_major=True)
    want = O.treeshap(model_io.forest_from_json(obj), obj["baseScore"], obj["numBins"], xs)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
