"""CPU tests of the shipped library: it loads, exports every symbol the header
declares, validates inputs with the reference's messages, and fails loudly
(never silently falls back) when no GPU is present."""
import json
import re
from pathlib import Path

import numpy as np
import pytest

import macboost_amd as mb
import model_io
import oracle_lib as O
from macboost_amd import _core

ROOT = Path(__file__).resolve().parent.parent


def _has_gpu():
    try:
        ctx = mb.Context(0)
        ctx.close()
        return True
    except mb.MacBoostError:
        return False


def test_exports_every_header_symbol():
    header = (ROOT / "include" / "macboost.h").read_text()
    declared = set(re.findall(r"\b((?:macboost|mbk|mbx)_[a-z_]+)\s*\(", header))
    declared -= {"mbk_context", "mbk_split_result"}
    lib = _core.lib()
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing
    assert declared == set(_core.EXPORTED)
    # the 14 reference entry points (CAPI.swift)
    assert len([s for s in declared if s.startswith("macboost_")]) == 14


@pytest.mark.parametrize("params,msg", [
    ({"num_bins": 3}, "Invalid input: numBins must be in 4...256, got 3"),
    ({"max_depth": 13}, "Invalid input: maxDepth must be in 1...12, got 13"),
    ({"num_trees": 0}, "Invalid input: numTrees must be >= 1, got 0"),
    ({"learning_rate": 0.0}, "Invalid input: learningRate must be positive and finite"),
    ({"objective": "nope"}, "Internal error: unknown objective 'nope'"),
    ({"num_leaves": 65}, "Invalid input: numLeaves must be in 2...2^maxDepth (= 64), got 65"),
    ({"metric": "auc"}, "Invalid input: auc metric requires the binary objective"),
    ({"goss": True, "goss_top_rate": 0.8, "goss_other_rate": 0.5},
     "Invalid input: GOSS rates must be positive with topRate + otherRate <= 1"),
])
def test_param_validation_messages(params, msg):
    # Booster.swift:262-330, CAPI.swift:63-73
    x = np.zeros((4, 2), np.float32)
    with pytest.raises(mb.MacBoostError) as e:
        mb.train(params, x, np.zeros(4, np.float32))
    assert str(e.value) == msg


def test_data_validation_messages():
    # Booster.swift:1724-1765, :1810-1826, CAPI.swift:97-99
    x = np.zeros((4, 1), np.float32)
    with pytest.raises(mb.MacBoostError, match="labels must be finite"):
        mb.train({}, x, np.array([0, 1, np.nan, 2], np.float32))
    with pytest.raises(mb.MacBoostError, match=r"binary objective requires labels in \{0, 1\}"):
        mb.train({"objective": "binary"}, x, np.array([0, 1, 2, 1], np.float32))
    with pytest.raises(mb.MacBoostError,
                       match=r"Categorical feature 0 has value 999.0; expected integer ids in "
                             r"0..<255 or NaN"):
        mb.train({"categorical_features": [0]}, np.array([[0], [1], [2], [999]], np.float32),
                 np.zeros(4, np.float32))
    with pytest.raises(mb.MacBoostError, match="weights must be finite and >= 0"):
        mb.train({}, x, np.zeros(4, np.float32), sample_weight=np.array([1, -1, 1, 1], np.float32))
    with pytest.raises(mb.MacBoostError, match="null or empty training data"):
        mb.train({}, np.zeros((0, 3), np.float32), np.zeros(0, np.float32))


@pytest.mark.skipif(_has_gpu(), reason="checks the no-GPU failure path")
def test_no_gpu_fails_loudly():
    x, y = O.friedman(500, 6, 1)
    with pytest.raises(mb.MacBoostError, match="No HIP GPU available"):
        mb.train({"num_trees": 2}, x, y, feature_major=True)
    with pytest.raises(mb.MacBoostError, match="No HIP GPU available"):
        mb.Context(0)


def test_friedman_generator_matches_oracle():
    # the library's multithreaded DataGen.friedman equals the oracle bit for bit
    x1, y1 = mb.friedman(70_000, 7, 42)
    x2, y2 = O.friedman(70_000, 7, 42)
    assert np.array_equal(x1, x2) and np.array_equal(y1, y2)


def _small_oracle_model():
    x, y = O.friedman(3000, 6, 5)
    m = O.fit_raw(x, y, num_bins=64, num_trees=4, max_depth=3)
    return x, m


def test_model_json_roundtrip_without_gpu(tmp_path):
    x, m = _small_oracle_model()
    obj = model_io.forest_to_json(m.forest, base=m.base_score, num_bins=64, num_features=6)
    p = tmp_path / "model.json"
    p.write_text(json.dumps(obj))
    h = mb.load(p)
    assert mb.num_trees(h) == 4 and mb.num_features(h) == 6 and mb.num_classes(h) == 1
    # feature importance (Booster.swift:1926-1940) on the host
    split = mb.feature_importance(h, "split")
    want = np.zeros(6, np.float32)
    for t in range(4):
        for f in m.forest.feature[t][m.forest.feature[t] >= 0]:
            want[f] += 1
    assert np.array_equal(split, want)
    q = tmp_path / "again.json"
    mb.save(h, q)
    again = json.loads(q.read_text())
    f2 = model_io.forest_from_json(again)
    model_io.assert_same_forest(m.forest, f2, with_cats=False)
    assert np.float32(again["baseScore"]) == np.float32(m.base_score)


def test_malformed_model_is_rejected(tmp_path):
    x, m = _small_oracle_model()
    obj = model_io.forest_to_json(m.forest, base=m.base_score, num_bins=64, num_features=6)
    obj["trees"][0]["feature"][-1] = 2            # a split with no children
    p = tmp_path / "bad.json"
    p.write_text(json.dumps(obj))
    with pytest.raises(mb.MacBoostError, match="split without children"):
        mb.load(p)
    obj = model_io.forest_to_json(m.forest, base=m.base_score, num_bins=64, num_features=6)
    obj["version"] = 2
    p.write_text(json.dumps(obj))
    with pytest.raises(mb.MacBoostError, match="unsupported model file"):
        mb.load(p)


def test_init_model_validation_without_gpu(tmp_path):
    # Booster.swift:487-499: the init model must match the features and
    # objective, and cannot seed a prebinned dataset
    x, m = _small_oracle_model()
    obj = model_io.forest_to_json(m.forest, base=m.base_score, num_bins=64, num_features=6)
    p = tmp_path / "init.json"
    p.write_text(json.dumps(obj))
    x5, y5 = O.friedman(500, 5, 3)
    with pytest.raises(mb.MacBoostError, match="initModel expects 6 features, X has 5"):
        mb.train({"init_model": str(p)}, x5, y5, feature_major=True)
    x6, y6 = O.friedman(500, 6, 3)
    with pytest.raises(mb.MacBoostError, match="initModel objective differs"):
        mb.train({"init_model": str(p), "objective": "huber"}, x6, y6, feature_major=True)
    with pytest.raises(mb.MacBoostError, match="cannot read"):
        mb.train({"init_model": str(tmp_path / "missing.json")}, x6, y6, feature_major=True)
    from oracle import mbds as M
    M.write(tmp_path / "d.mbds", 500, 6, 64, [], None, np.zeros((6, 62), np.float32), y6,
            M.tile8(np.zeros((6, 500), np.uint8)))
    ds = mb.Dataset.load(tmp_path / "d.mbds")
    with pytest.raises(mb.MacBoostError,
                       match=r"initModel requires raw features \(not a prebinned dataset\)"):
        mb.train_dataset({"init_model": str(p)}, ds)


def test_select_features_validation_without_gpu():
    # FeatureSelection.swift:53-69, CAPI.swift:150-152
    x, y = O.friedman(200, 6, 1)
    with pytest.raises(mb.MacBoostError,
                       match=r"Invalid input: selection needs rounds >= 5 for the binomial test"):
        mb.select_features({}, x, y, rounds=4, feature_major=True)
    with pytest.raises(mb.MacBoostError, match=r"Invalid input: alpha must be in \(0, 1\)"):
        mb.select_features({}, x, y, alpha=1.5, feature_major=True)
    with pytest.raises(mb.MacBoostError, match="binary objective requires labels"):
        mb.select_features({"objective": "binary"}, x, y, feature_major=True)
    h = np.empty(6, np.int32)
    err = _core.ctypes.c_char_p()
    rc = _core.lib().macboost_select_features(b"{}", None, 200, 6, None, None, 20, 0, 0.05, 0,
                                              h.ctypes.data_as(_core.ctypes.POINTER(_core.ctypes.c_int32)),
                                              h.ctypes.data_as(_core.ctypes.POINTER(_core.ctypes.c_int32)),
                                              None, _core.ctypes.byref(err))
    assert rc == 1 and b"null or empty selection input" in err.value


def _no_library(monkeypatch):
    def refuse():
        raise AssertionError("the library was called before the inputs were checked")
    monkeypatch.setattr(_core, "lib", refuse)


@pytest.mark.parametrize("case,msg", [
    ("short_y", "y has 9 rows, X has 10"),
    ("long_y", "y has 11 rows, X has 10"),
    ("short_w", "sample_weight has 3 rows, X has 10"),
    ("eval_cols", "eval_set feature count differs from X"),
    ("eval_rows", "eval_set X/y row mismatch"),
    ("x_1d", "X must be 2-dimensional, got shape (10,)"),
])
def test_shape_checks_before_any_library_call(monkeypatch, case, msg):
    # python/macboost/_core.py:149-167: the binding checks y, sample_weight
    # and eval_set against X before the library reads rows * cols floats
    x = np.zeros((10, 3), np.float32)
    y = np.zeros(10, np.float32)
    kw = {}
    if case == "short_y":
        y = y[:9]
    elif case == "long_y":
        y = np.zeros(11, np.float32)
    elif case == "short_w":
        kw["sample_weight"] = np.ones(3, np.float32)
    elif case == "eval_cols":
        kw["eval_set"] = (np.zeros((5, 2), np.float32), np.zeros(5, np.float32))
    elif case == "eval_rows":
        kw["eval_set"] = (np.zeros((5, 3), np.float32), np.zeros(4, np.float32))
    elif case == "x_1d":
        x = np.zeros(10, np.float32)
    _no_library(monkeypatch)
    for call in (mb.train, mb.Trainer):
        with pytest.raises(ValueError) as e:
            call({"num_trees": 1}, x, y, **kw)
        assert str(e.value) == msg
    if case in ("short_y", "long_y", "x_1d"):
        with pytest.raises(ValueError):
            mb.Dataset.make({}, x, y)


def test_labels_are_raveled(monkeypatch):
    # a (rows, 1) label column is accepted as rows labels
    cfg, xf, rows, cols, rm, yv, w, xv, vrows, yvv = _core._prep_train(
        {}, np.zeros((6, 2), np.float32), np.zeros((6, 1), np.float32),
        (np.zeros((4, 2), np.float32), np.zeros((4, 1), np.float32)), np.ones((6, 1)))
    assert yv.shape == (6,) and w.shape == (6,) and yvv.shape == (4,) and xv.shape == (2, 4)
    assert (rows, cols, rm, vrows) == (6, 2, 1, 4)
