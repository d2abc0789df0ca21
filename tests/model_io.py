"""Model-file helpers shared by tests: the reference's model JSON
(Booster.swift:2119-2162) <-> the oracle's flat forest arrays."""
import json
import tempfile
from pathlib import Path

import numpy as np

import oracle_lib as O


def forest_from_json(obj: dict, nodes: int | None = None) -> O.Forest:
    trees = obj["trees"]
    nodes = nodes or max(len(t["feature"]) for t in trees)
    has_cats = any(len(t["catMask"]) for t in trees)
    f = O.Forest.empty(len(trees), nodes, with_cats=has_cats)
    for i, t in enumerate(trees):
        n = len(t["feature"])
        f.feature[i, :n] = t["feature"]
        f.threshold[i, :n] = np.array(t["threshold"], np.float32)
        f.leaf[i, :n] = np.array(t["leaf"], np.float32)
        f.flags[i, :n] = t["flags"]
        f.gain[i, :n] = np.array(t.get("gain", [0] * n), np.float32)
        f.cover[i, :n] = np.array(t.get("cover", [0] * n), np.float32)
        if has_cats and t["catMask"]:
            f.cat_mask[i, :n] = np.array(t["catMask"], np.uint32).reshape(n, 8)
    return f


def forest_to_json(f: O.Forest, *, base: float, num_bins: int, num_features: int,
                   categorical=(), with_cats=None) -> dict:
    with_cats = bool(categorical) if with_cats is None else with_cats
    trees = []
    for i in range(f.num_trees):
        trees.append({
            "feature": f.feature[i].tolist(),
            "threshold": [float(v) for v in f.threshold[i]],
            "leaf": [float(v) for v in f.leaf[i]],
            "flags": f.flags[i].tolist(),
            "catMask": f.cat_mask[i].reshape(-1).tolist() if with_cats else [],
            "gain": [float(v) for v in f.gain[i]],
            "cover": [float(v) for v in f.cover[i]],
        })
    return {"version": 1, "objective": 0, "numBins": num_bins, "baseScore": float(base),
            "numFeatures": num_features, "categorical": list(categorical), "trees": trees,
            "numClasses": 1, "baseScores": [float(base)]}


def saved_model(handle) -> dict:
    import macboost_amd as mb
    with tempfile.TemporaryDirectory() as d:
        p = Path(d) / "m.json"
        mb.save(handle, p)
        return json.loads(p.read_text())


def assert_same_forest(a: O.Forest, b: O.Forest, with_cats: bool):
    for name in ("feature", "threshold", "leaf", "flags", "gain", "cover"):
        x, y = getattr(a, name), getattr(b, name)
        assert x.shape == y.shape, name
        if not np.array_equal(x, y):
            bad = np.argwhere(x != y)[:5]
            raise AssertionError(f"{name} differs at {bad.tolist()}: "
                                 f"{[x[tuple(i)] for i in bad]} vs {[y[tuple(i)] for i in bad]}")
    if with_cats:
        assert np.array_equal(a.cat_mask, b.cat_mask), "cat_mask"
