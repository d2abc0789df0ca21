"""MI355X (gfx950) build of MacBoost's on-device tree-build path.

The compute lives in ``libmacboostc.so`` (HIP kernels + C++ host, built from
``macboost_amd/csrc``); this package is its ctypes front end, with the same
entry points as the reference binding (python/macboost/_core.py).
"""
from ._core import (  # noqa: F401
    Context, Dataset, MacBoostError, Trainer, best_iteration, eval_history,
    feature_importance, friedman,
    load, num_classes, num_features, num_trees, predict, predict_contrib, profile_train, save,
    select_features, train, train_dataset, train_hist_stats, version, warnings,
)
