"""Preprocessed datasets (.mbds): the file format (Dataset.swift:26-86) on the
CPU, and makeDataset / fit(dataset:) (Booster.swift:375-436) on the GPU.

The CPU tests pin the numpy restatement of the format (oracle/mbds.py) with a
hand-assembled file, then check that the library reads what it writes and
writes byte for byte what it reads.  The GPU tests check the device-built
dataset against the oracle's edges and bins, and that training from a saved
and reloaded dataset gives the same model as training from the raw matrix
(the reference allows an RMSE difference of 0.03, FeatureTests.swift:238-277;
this path is deterministic, so the models are identical).
"""
import struct

import numpy as np
import pytest

import macboost_amd as mb
import model_io
import oracle_lib as O
from macboost_amd import _core
from oracle import mbds as M


def _random_dataset(rows, cols, nb, seed, names=True):
    rng = np.random.default_rng(seed)
    cats = sorted(rng.choice(cols, size=min(2, cols), replace=False).tolist())
    fm = rng.integers(0, nb, size=(cols, rows), dtype=np.uint8)
    edges = np.sort(rng.standard_normal((cols, nb - 2)).astype(np.float32), axis=1)
    labels = rng.standard_normal(rows).astype(np.float32)
    fn = [f"f/{i}" for i in range(cols)] if names else None
    return dict(rows=rows, cols=cols, num_bins=nb, categorical=cats, feature_names=fn,
                edges=edges, labels=labels, bins=M.tile8(fm))


def test_format_restatement_known_bytes(tmp_path):
    # One row, two features, 4 bins, feature 1 categorical, names ["a/b", "c"]:
    # every field assembled by hand from Dataset.swift:26-41.
    want = (b"SDBM" + bytes([1, 0, 0, 0]) + bytes([8, 0, 0, 0])
            + bytes([1, 0, 0, 0, 0, 0, 0, 0])            # rows
            + bytes([2, 0, 0, 0]) + bytes([4, 0, 0, 0])  # cols, numBins
            + bytes([1, 0, 0, 0]) + bytes([1, 0, 0, 0])  # one categorical: 1
            + bytes([12, 0, 0, 0]) + b'["a\\/b","c"]'    # JSONEncoder escapes '/'
            + bytes([4, 0, 0, 0, 0, 0, 0, 0])            # 2 cols x 2 edges
            + bytes.fromhex("0000803f" "00000040" "00000000" "00000000")   # 1, 2, 0, 0
            + bytes([1, 0, 0, 0, 0, 0, 0, 0]) + bytes.fromhex("0000c0bf")  # label -1.5
            + bytes([8, 0, 0, 0, 0, 0, 0, 0]) + bytes([3, 1, 0, 0, 0, 0, 0, 0]))
    got = M.write(tmp_path / "k.mbds", 1, 2, 4, [1], ["a/b", "c"],
                  np.array([[1, 2], [0, 0]], np.float32), np.array([-1.5], np.float32),
                  M.tile8(np.array([[3], [1]], np.uint8)))
    assert got == want


def test_tile8_layout_matches_bin_index():
    # bin_index (Shaders.swift:37-39): (f >> 3) * n * 8 + i * 8 + (f & 7)
    rows, cols = 5, 11
    fm = np.arange(cols * rows, dtype=np.uint8).reshape(cols, rows)
    flat = M.tile8(fm).ravel()
    for f in range(cols):
        for i in range(rows):
            assert flat[(f >> 3) * rows * 8 + i * 8 + (f & 7)] == fm[f, i]
    assert flat.size == 2 * rows * 8 and not M.tile8(fm)[1, :, 3:].any()


@pytest.mark.parametrize("rows,cols,nb,names", [(1, 1, 4, False), (37, 9, 64, True),
                                                 (1000, 17, 256, True)])
def test_library_reads_and_rewrites_oracle_files(tmp_path, rows, cols, nb, names):
    d = _random_dataset(rows, cols, nb, rows + cols, names)
    want = M.write(tmp_path / "a.mbds", **d)
    ds = mb.Dataset.load(tmp_path / "a.mbds")
    assert (ds.rows, ds.cols, ds.num_bins) == (rows, cols, nb)
    cat, labels, edges, bins = ds.arrays()
    assert cat.tolist() == d["categorical"]
    assert np.array_equal(labels, d["labels"])
    assert np.array_equal(edges, d["edges"])
    assert np.array_equal(bins, d["bins"])
    assert ds.feature_names == d["feature_names"]
    ds.save(tmp_path / "b.mbds")
    assert (tmp_path / "b.mbds").read_bytes() == want


def _expect_load_error(path, msg):
    with pytest.raises(mb.MacBoostError) as e:
        mb.Dataset.load(path)
    assert str(e.value) == msg


def test_load_errors(tmp_path):
    # Dataset.swift:47-84, with the C ABI's "Invalid input: " prefix
    d = _random_dataset(20, 10, 16, 3)
    good = M.write(tmp_path / "g.mbds", **d)
    cases = {
        "trunc": (good[:-1], "Invalid input: truncated .mbds file"),
        "empty": (b"", "Invalid input: truncated .mbds file"),
        "magic": (b"XDBM" + good[4:], "Invalid input: not a MacBoost dataset (.mbds) file"),
        "version": (good[:4] + struct.pack("<I", 2) + good[8:],
                    "Invalid input: unsupported .mbds version"),
        "tile": (good[:8] + struct.pack("<I", 16) + good[12:],
                 "Invalid input: .mbds tile width mismatch"),
    }
    for name, (data, msg) in cases.items():
        p = tmp_path / f"{name}.mbds"
        p.write_bytes(data)
        _expect_load_error(p, msg)
    bad = dict(d, labels=d["labels"][:-1])                 # labelCount != rows
    M.write(tmp_path / "l.mbds", **bad)
    _expect_load_error(tmp_path / "l.mbds", "Invalid input: .mbds sizes are inconsistent")
    bad = dict(d, edges=d["edges"][:, :-1])                # edgeCount != cols*(numBins-2)
    M.write(tmp_path / "e.mbds", **bad)
    _expect_load_error(tmp_path / "e.mbds", "Invalid input: .mbds sizes are inconsistent")
    bad = dict(d, categorical=[3, 10])                     # index past the last feature
    M.write(tmp_path / "c.mbds", **bad)
    _expect_load_error(tmp_path / "c.mbds",
                       "Invalid input: .mbds categorical feature index out of range")
    with pytest.raises(mb.MacBoostError):
        mb.Dataset.load(tmp_path / "missing.mbds")


def test_null_dataset_handles():
    lib = _core.lib()
    assert lib.mbx_dataset_info(None, None, None, None, None) == -1
    assert lib.mbx_dataset_copy(None, None, None, None, None) == -1
    assert lib.mbx_dataset_feature_names(None) is None
    lib.mbx_dataset_free(None)


# --------------------------------------------------------------------------
# GPU: makeDataset and fit(dataset:)
# --------------------------------------------------------------------------

def _mixed(rows, seed):
    x, y = O.friedman(rows, 8, seed)
    rng = O.SplitMix(seed + 1)
    miss = O.SplitMix(seed + 2).uniforms(rows) < 0.1
    x[2][miss] = np.nan
    cat = np.array([rng.next() % 5 for _ in range(rows)], np.float32)
    x = np.vstack([x, cat[None, :]])
    y = (y + np.where(cat == 2, 3.0, 0.0)).astype(np.float32)
    return x, y


@pytest.mark.gpu
def test_make_dataset_matches_oracle():
    rows, nb = 20_000, 64
    x, y = _mixed(rows, 71)
    is_cat = np.zeros(9, np.uint8)
    is_cat[8] = 1
    names = [f"c{i}" for i in range(9)]
    ds = mb.Dataset.make({"num_bins": nb, "categorical_features": [8]}, x, y, names,
                         feature_major=True)
    cat, labels, edges, bins = ds.arrays()
    want_edges = O.compute_edges(x, nb, is_cat)
    assert cat.tolist() == [8]
    assert np.array_equal(labels, y)
    assert np.array_equal(edges, want_edges)
    assert np.array_equal(bins, M.tile8(O.bin_matrix(x, want_edges, nb, is_cat)))
    assert ds.feature_names == names
    # row-major input gives the same dataset
    ds2 = mb.Dataset.make({"num_bins": nb, "categorical_features": [8]},
                          np.ascontiguousarray(x.T), y, names)
    assert all(np.array_equal(a, b) for a, b in zip(ds.arrays(), ds2.arrays()))


@pytest.mark.gpu
def test_train_from_saved_dataset_equals_raw(tmp_path):
    # FeatureTests.swift:238-277: makeDataset -> save -> load -> fit(dataset:)
    # with a fresh booster that has NO categorical params (the dataset's
    # layout must win) against fit on the raw matrix.
    rows = 20_000
    x, y = _mixed(rows, 71)
    p = {"num_trees": 60, "max_depth": 5, "categorical_features": [8]}
    names = [f"c{i}" for i in range(9)]
    ds = mb.Dataset.make(p, x, y, names, feature_major=True)
    ds.save(tmp_path / "d.mbds")
    loaded = mb.Dataset.load(tmp_path / "d.mbds")
    assert all(np.array_equal(a, b) for a, b in zip(ds.arrays(), loaded.arrays()))
    h_ds = mb.train_dataset({"num_trees": 60, "max_depth": 5}, loaded)
    h_raw = mb.train(p, x, y, feature_major=True)
    a, b = model_io.saved_model(h_ds), model_io.saved_model(h_raw)
    fa = model_io.forest_from_json(a, 63)
    fb = model_io.forest_from_json(b, 63)
    model_io.assert_same_forest(fa, fb, with_cats=True)
    assert np.array_equal(mb.predict(h_ds, x, feature_major=True),
                          mb.predict(h_raw, x, feature_major=True))
    assert a["featureNames"] == names
    assert (fa.flags & O.FLAG_CATEGORICAL).any()


@pytest.mark.gpu
def test_train_from_dataset_with_validation_and_weights():
    rows = 12_000
    x, y = _mixed(rows, 5)
    xv, yv = _mixed(3000, 6)
    w = np.linspace(0.5, 1.5, rows).astype(np.float32)
    p = {"num_trees": 40, "max_depth": 6, "num_bins": 128, "categorical_features": [8],
         "early_stopping_rounds": 5}
    ds = mb.Dataset.make(p, x, y, feature_major=True)
    h_ds = mb.train_dataset(p, ds, eval_set=(xv.T, yv), sample_weight=w)
    h_raw = mb.train(p, x, y, eval_set=(xv.T, yv), sample_weight=w, feature_major=True)
    assert mb.best_iteration(h_ds) == mb.best_iteration(h_raw)
    assert np.array_equal(mb.predict(h_ds, xv, feature_major=True),
                          mb.predict(h_raw, xv, feature_major=True))
