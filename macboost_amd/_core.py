"""ctypes binding to libmacboostc.so, the MI355X build of MacBoost's C ABI.

Mirrors the reference binding (python/macboost/_core.py): the same symbols,
argtypes (_core.py:59-96), the row-major fast path of ``train``
(_core.py:135-177), feature-major ``predict``/``predict_contrib``
(_core.py:210-231) and error-string ownership (_core.py:103-107).  The
library is loaded from this package directory; when it is missing every call
raises — there is no pure-Python fallback.
"""
from __future__ import annotations

import ctypes
import json
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libmacboostc.so"

_c_char_pp = ctypes.POINTER(ctypes.c_char_p)
_f32_p = ctypes.POINTER(ctypes.c_float)
_P = ctypes.c_void_p

_lib_instance = None


class MacBoostError(RuntimeError):
    pass


def _find_library() -> str:
    env = os.environ.get("MACBOOST_LIB")
    for c in ([Path(env)] if env else []) + [LIB_PATH]:
        if c.is_file():
            return str(c)
    raise OSError(f"{LIB_PATH} not found; build it with `make -C macboost_amd/csrc` "
                  "(or __graft_entry__.build())")


def lib() -> ctypes.CDLL:
    global _lib_instance
    if _lib_instance is None:
        _lib_instance = ctypes.CDLL(_find_library())
        _configure(_lib_instance)
    return _lib_instance


class MbkTreeShape(ctypes.Structure):
    """mbk_tree_shape (include/macboost.h)."""
    _fields_ = [("rows", ctypes.c_int64), ("cols", ctypes.c_int32),
                ("num_bins", ctypes.c_int32), ("tile_width", ctypes.c_int32),
                ("max_depth", ctypes.c_int32)]


class MbkSplitParams(ctypes.Structure):
    """mbk_split_params (include/macboost.h)."""
    _fields_ = [("lambda_", ctypes.c_float), ("min_child_hess", ctypes.c_float),
                ("min_split_gain", ctypes.c_float), ("cat_smooth", ctypes.c_float),
                ("learning_rate", ctypes.c_float)]


class MbkTreeOut(ctypes.Structure):
    """mbk_tree_out: device pointers of one tree's model arrays."""
    _fields_ = [("split", _P), ("leaf", _P), ("gain", _P), ("cover", _P), ("mask", _P)]


_SHAPE_P = ctypes.POINTER(MbkTreeShape)
_SPLIT_P = ctypes.POINTER(MbkSplitParams)


def _configure(l):
    l.macboost_train.restype = ctypes.c_void_p
    l.macboost_train.argtypes = [
        ctypes.c_char_p, _f32_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
        _f32_p, _f32_p, _f32_p, ctypes.c_int64, _f32_p, _c_char_pp,
    ]
    l.macboost_select_features.restype = ctypes.c_int32
    l.macboost_select_features.argtypes = [
        ctypes.c_char_p, _f32_p, ctypes.c_int64, ctypes.c_int64, _f32_p, _f32_p,
        ctypes.c_int32, ctypes.c_int32, ctypes.c_float, ctypes.c_int64,
        ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32), _f32_p, _c_char_pp,
    ]
    l.macboost_predict_contrib.restype = ctypes.c_int32
    l.macboost_predict_contrib.argtypes = [
        ctypes.c_void_p, _f32_p, ctypes.c_int64, ctypes.c_int64, _f32_p, _c_char_pp,
    ]
    l.macboost_feature_importance.restype = ctypes.c_int32
    l.macboost_feature_importance.argtypes = [ctypes.c_void_p, ctypes.c_int32, _f32_p]
    l.macboost_predict.restype = ctypes.c_int32
    l.macboost_predict.argtypes = [
        ctypes.c_void_p, _f32_p, ctypes.c_int64, ctypes.c_int64, _f32_p, _c_char_pp,
    ]
    l.macboost_save.restype = ctypes.c_int32
    l.macboost_save.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _c_char_pp]
    l.macboost_load.restype = ctypes.c_void_p
    l.macboost_load.argtypes = [ctypes.c_char_p, _c_char_pp]
    for name in ("macboost_num_trees", "macboost_num_features", "macboost_best_iteration",
                 "macboost_num_classes"):
        fn = getattr(l, name)
        fn.restype = ctypes.c_int64
        fn.argtypes = [ctypes.c_void_p]
    l.macboost_warnings.restype = ctypes.c_void_p
    l.macboost_warnings.argtypes = [ctypes.c_void_p]
    l.macboost_free.restype = None
    l.macboost_free.argtypes = [ctypes.c_void_p]
    l.macboost_free_string.restype = None
    l.macboost_free_string.argtypes = [ctypes.c_void_p]
    # kernel seam
    l.mbk_context_create.restype = ctypes.c_int
    l.mbk_context_create.argtypes = [ctypes.c_int32, ctypes.POINTER(_P), _c_char_pp]
    l.mbk_context_destroy.restype = None
    l.mbk_context_destroy.argtypes = [_P]
    l.mbk_device_alloc.restype = ctypes.c_int
    l.mbk_device_alloc.argtypes = [_P, ctypes.c_size_t, ctypes.POINTER(_P), _c_char_pp]
    l.mbk_device_free.restype = None
    l.mbk_device_free.argtypes = [_P, _P]
    for n in ("mbk_copy_to_device", "mbk_copy_to_host"):
        getattr(l, n).restype = ctypes.c_int
        getattr(l, n).argtypes = [_P, _P, _P, ctypes.c_size_t, _c_char_pp]
    l.mbk_synchronize.restype = ctypes.c_int
    l.mbk_synchronize.argtypes = [_P, _c_char_pp]
    l.mbk_quantile_edges.restype = ctypes.c_int
    l.mbk_quantile_edges.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int32, _P, _P, _c_char_pp]
    l.mbk_bin_data.restype = ctypes.c_int
    l.mbk_bin_data.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                               ctypes.c_int64, _P, _P, ctypes.c_int32, ctypes.c_int32, _P, _P,
                               _c_char_pp]
    l.mbk_quantize.restype = ctypes.c_int
    l.mbk_quantize.argtypes = [_P, ctypes.c_int32, ctypes.c_float, ctypes.c_float, _P, _P, _P,
                               ctypes.c_int64, _P, _P, _c_char_pp]
    l.mbk_node_hist_split.restype = ctypes.c_int
    l.mbk_node_hist_split.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_int32, _P, ctypes.c_int64, _P, _P, _P,
                                      ctypes.c_float, ctypes.c_float, ctypes.c_float, _P, _P,
                                      _c_char_pp]
    for name, args in (
            ("mbk_tree_begin", [_P, _SHAPE_P, _P, ctypes.c_int64, MbkTreeOut, _c_char_pp]),
            ("mbk_hist_build", [_P, ctypes.c_int32, _P, _P, _P, _c_char_pp]),
            ("mbk_hist_subtract", [_P, ctypes.c_int32, _P, _P, _c_char_pp]),
            ("mbk_find_splits", [_P, ctypes.c_int32, _P, _P, _P, _P, _SPLIT_P, _P, _c_char_pp]),
            ("mbk_decide_level", [_P, ctypes.c_int32, _P, _P, _SPLIT_P, MbkTreeOut,
                                  _c_char_pp]),
            ("mbk_route", [_P, ctypes.c_int32, _P, _P, _P, MbkTreeOut, _c_char_pp]),
            ("mbk_final_leaves", [_P, _P, _SPLIT_P, MbkTreeOut, _P, _c_char_pp]),
            ("mbk_grow_tree", [_P, _SHAPE_P, _SPLIT_P, _P, _P, _P, _P, _P, _P, _P, _P,
                               ctypes.c_int64, _P, _P, _P, MbkTreeOut, _P, _c_char_pp]),
            ("mbk_treeshap", [_P, _P, _P, _P, _P, _P, _P, ctypes.c_int32, ctypes.c_int32,
                              ctypes.c_float, ctypes.c_int32, _P, ctypes.c_int64, ctypes.c_int32,
                              _P, _c_char_pp])):
        getattr(l, name).restype = ctypes.c_int
        getattr(l, name).argtypes = args
    l.mbk_fit.restype = ctypes.c_void_p
    l.mbk_fit.argtypes = [_P, ctypes.c_char_p, _P, ctypes.c_int64, ctypes.c_int64,
                          ctypes.c_int32, _f32_p, _f32_p, _f32_p, ctypes.c_int64, _f32_p,
                          _c_char_pp]
    l.mbk_node_hist_split_noalloc.restype = ctypes.c_int
    l.mbk_node_hist_split_noalloc.argtypes = l.mbk_node_hist_split.argtypes
    l.mbk_predict_forest.restype = ctypes.c_int
    l.mbk_predict_forest.argtypes = [_P, _P, _P, _P, _P, _P, ctypes.c_int32, ctypes.c_int32, _P,
                                     ctypes.c_int64, ctypes.c_int32, ctypes.c_float, _P,
                                     _c_char_pp]
    # extensions
    l.mbx_trainer_create.restype = ctypes.c_void_p
    l.mbx_trainer_create.argtypes = l.macboost_train.argtypes
    l.mbx_trainer_grow.restype = ctypes.c_int
    l.mbx_trainer_grow.argtypes = [_P, ctypes.c_int32, _c_char_pp]
    l.mbx_trainer_profile.restype = ctypes.c_int
    l.mbx_trainer_profile.argtypes = [_P, ctypes.c_int32, _c_char_pp]
    l.mbx_trainer_hist_stats.restype = ctypes.c_int
    l.mbx_trainer_hist_stats.argtypes = [_P, ctypes.POINTER(ctypes.c_int64),
                                         ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(ctypes.c_double), _c_char_pp]
    l.mbx_trainer_level_stats.restype = ctypes.c_int
    l.mbx_trainer_level_stats.argtypes = [_P, ctypes.c_int32, _P, _P, _P, _c_char_pp]
    l.mbx_trainer_setup_seconds.restype = ctypes.c_int
    l.mbx_trainer_setup_seconds.argtypes = [_P, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_double)]
    l.mbx_trainer_booster.restype = ctypes.c_void_p
    l.mbx_trainer_booster.argtypes = [_P, _c_char_pp]
    l.mbx_trainer_free.restype = None
    l.mbx_trainer_free.argtypes = [_P]
    l.mbx_friedman.restype = None
    l.mbx_friedman.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64, ctypes.c_float,
                               _P, _P]
    l.mbx_context_profile.restype = ctypes.c_int
    l.mbx_context_profile.argtypes = [_P, ctypes.c_int32, _c_char_pp]
    l.mbx_context_hist_stats.restype = ctypes.c_int
    l.mbx_context_hist_stats.argtypes = [_P, ctypes.c_int32, ctypes.POINTER(ctypes.c_int64),
                                         ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(ctypes.c_double), _P, _P, _c_char_pp]
    l.mbx_profile_global.restype = ctypes.c_int
    l.mbx_profile_global.argtypes = [ctypes.c_int32, _c_char_pp]
    l.mbx_profile_global_stats.restype = ctypes.c_int
    l.mbx_profile_global_stats.argtypes = [ctypes.c_int32, ctypes.POINTER(ctypes.c_int64),
                                           ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_double), _P, _P, _c_char_pp]
    l.mbx_eval_history.restype = ctypes.c_int64
    l.mbx_eval_history.argtypes = [_P, _P, ctypes.c_int64]
    l.mbx_version.restype = ctypes.c_char_p
    l.mbx_version.argtypes = []
    l.mbx_dataset_make.restype = ctypes.c_void_p
    l.mbx_dataset_make.argtypes = [ctypes.c_char_p, _P, ctypes.c_int64, ctypes.c_int64,
                                   ctypes.c_int32, _P, ctypes.c_char_p, _c_char_pp]
    l.mbx_dataset_save.restype = ctypes.c_int32
    l.mbx_dataset_save.argtypes = [_P, ctypes.c_char_p, _c_char_pp]
    l.mbx_dataset_load.restype = ctypes.c_void_p
    l.mbx_dataset_load.argtypes = [ctypes.c_char_p, _c_char_pp]
    l.mbx_dataset_info.restype = ctypes.c_int32
    l.mbx_dataset_info.argtypes = [_P, ctypes.POINTER(ctypes.c_int64),
                                   ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_int32)]
    l.mbx_dataset_copy.restype = ctypes.c_int32
    l.mbx_dataset_copy.argtypes = [_P, _P, _P, _P, _P]
    l.mbx_dataset_feature_names.restype = ctypes.c_void_p
    l.mbx_dataset_feature_names.argtypes = [_P]
    l.mbx_dataset_train.restype = ctypes.c_void_p
    l.mbx_dataset_train.argtypes = [ctypes.c_char_p, _P, _P, _P, ctypes.c_int64, _P, _c_char_pp]
    l.mbx_dataset_free.restype = None
    l.mbx_dataset_free.argtypes = [_P]


EXPORTED = (
    "macboost_train", "macboost_select_features", "macboost_predict", "macboost_num_classes",
    "macboost_feature_importance", "macboost_predict_contrib", "macboost_save", "macboost_load",
    "macboost_num_trees", "macboost_num_features", "macboost_best_iteration",
    "macboost_warnings", "macboost_free", "macboost_free_string",
    "mbk_context_create", "mbk_context_destroy", "mbk_device_alloc", "mbk_device_free",
    "mbk_copy_to_device", "mbk_copy_to_host", "mbk_synchronize", "mbk_quantile_edges", "mbk_bin_data", "mbk_quantize",
    "mbk_node_hist_split", "mbk_predict_forest", "mbk_fit", "mbk_tree_begin", "mbk_hist_build",
    "mbk_hist_subtract", "mbk_find_splits", "mbk_decide_level", "mbk_route", "mbk_final_leaves",
    "mbk_grow_tree", "mbk_treeshap", "mbk_node_hist_split_noalloc",
    "mbx_trainer_create", "mbx_trainer_grow", "mbx_trainer_profile", "mbx_trainer_hist_stats",
    "mbx_trainer_level_stats", "mbx_trainer_setup_seconds", "mbx_trainer_booster", "mbx_trainer_free", "mbx_friedman",
    "mbx_version", "mbx_dataset_make", "mbx_dataset_save", "mbx_dataset_load",
    "mbx_dataset_info", "mbx_dataset_copy", "mbx_dataset_feature_names", "mbx_dataset_train",
    "mbx_dataset_free", "mbx_eval_history", "mbx_context_profile", "mbx_context_hist_stats",
    "mbx_profile_global", "mbx_profile_global_stats",
)


def _take_error(err: ctypes.c_char_p) -> str:
    """The library's malloc'd error text; the C string is released here."""
    text = (err.value or b"unknown error").decode()
    lib().macboost_free_string(ctypes.cast(err, ctypes.c_void_p))
    return text


def _matrix(X, name="X") -> np.ndarray:
    m = np.asarray(X, dtype=np.float32)
    if m.ndim != 2:
        raise ValueError(f"{name} must be 2-dimensional, got shape {m.shape}")
    return m


def _feature_major(X):
    """A (rows, cols) matrix as a contiguous [cols][rows] float32 copy."""
    m = _matrix(X)
    return np.ascontiguousarray(m.T), m.shape[0], m.shape[1]


def _column(v, rows: int, what: str) -> np.ndarray:
    """A label or weight vector: float32, flattened, one value per row."""
    a = np.ascontiguousarray(np.asarray(v, dtype=np.float32).ravel())
    if a.shape[0] != rows:
        raise ValueError(f"{what} has {a.shape[0]} rows, X has {rows}")
    return a


def _f32(a):
    return None if a is None else a.ctypes.data_as(_f32_p)


class _Handle:
    """A booster handle; the booster is released with the Python object."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    def __del__(self):
        ptr, self.ptr = getattr(self, "ptr", None), None
        if ptr and _lib_instance is not None:
            _lib_instance.macboost_free(ptr)


def _eval_arrays(eval_set, cols: int):
    """(feature-major X, y, rows) of a validation set, shape-checked against
    the training matrix (the library reads rows*cols and rows floats)."""
    if eval_set is None:
        return None, None, 0
    xv, yv = eval_set
    xf, vrows, vcols = _feature_major(xv)
    if vcols != cols:
        raise ValueError("eval_set feature count differs from X")
    ya = np.ascontiguousarray(np.asarray(yv, dtype=np.float32).ravel())
    if ya.shape[0] != vrows:
        raise ValueError("eval_set X/y row mismatch")
    return xf, ya, vrows


def _prep_train(config, X, y, eval_set, sample_weight, layout_fm=False):
    """Every input of macboost_train, checked before the library reads it:
    X is (rows, cols) row-major, or (cols, rows) with layout_fm."""
    m = _matrix(X)
    xf = np.ascontiguousarray(m)
    if layout_fm:
        cols, rows = xf.shape
    else:
        rows, cols = xf.shape
    yv = _column(y, rows, "y")
    w = None if sample_weight is None else _column(sample_weight, rows, "sample_weight")
    xv, yvv, vrows = _eval_arrays(eval_set, cols)
    cfg = json.dumps(config).encode()
    return cfg, xf, rows, cols, 0 if layout_fm else 1, yv, w, xv, vrows, yvv


def train(config: dict, X, y, eval_set=None, sample_weight=None, feature_major=False) -> _Handle:
    """macboost_train; X is (rows, cols) row-major, or (cols, rows) with feature_major."""
    cfg, xf, rows, cols, rm, yv, w, xv, vrows, yvv = _prep_train(
        config, X, y, eval_set, sample_weight, feature_major)
    err = ctypes.c_char_p()
    ptr = lib().macboost_train(cfg, _f32(xf), rows, cols, rm, _f32(yv), _f32(w), _f32(xv),
                               vrows, _f32(yvv), ctypes.byref(err))
    if not ptr:
        raise MacBoostError(_take_error(err))
    return _Handle(ptr)


def select_features(config: dict, X, y, sample_weight=None, rounds: int = 20, trees: int = 0,
                    alpha: float = 0.05, seed: int = 0, feature_major=False):
    """macboost_select_features (Boruta, CAPI.swift:138-183): (hits, decision
    2 confirmed / 1 tentative / 0 rejected, gain ratio) per feature."""
    xf, rows, cols = _as_feature_major(X, feature_major)
    ya = _column(y, rows, "y")
    wa = None if sample_weight is None else _column(sample_weight, rows, "sample_weight")
    hits = np.empty(cols, np.int32)
    decision = np.empty(cols, np.int32)
    ratio = np.empty(cols, np.float32)
    err = ctypes.c_char_p()
    rc = lib().macboost_select_features(
        json.dumps(config).encode(), _f32(xf), rows, cols, _f32(ya), _f32(wa), rounds, trees,
        alpha, seed, hits.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
        decision.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), _f32(ratio), ctypes.byref(err))
    if rc != 0:
        raise MacBoostError(_take_error(err))
    return hits, decision, ratio


def _as_feature_major(X, feature_major):
    """(contiguous [cols][rows] float32, rows, cols) from either layout."""
    if feature_major:
        xf = np.ascontiguousarray(_matrix(X))
        return xf, xf.shape[1], xf.shape[0]
    return _feature_major(X)


def predict(handle: _Handle, X, feature_major=False) -> np.ndarray:
    xf, rows, cols = _as_feature_major(X, feature_major)
    k = max(1, num_classes(handle))
    out = np.empty(rows * k, dtype=np.float32)
    err = ctypes.c_char_p()
    if lib().macboost_predict(handle.ptr, _f32(xf), rows, cols, _f32(out), ctypes.byref(err)) != 0:
        raise MacBoostError(_take_error(err))
    return out if k == 1 else out.reshape(rows, k)


def predict_contrib(handle: _Handle, X, feature_major=False) -> np.ndarray:
    xf, rows, cols = _as_feature_major(X, feature_major)
    k = max(1, num_classes(handle))
    out = np.empty(rows * k * (cols + 1), dtype=np.float32)
    err = ctypes.c_char_p()
    if lib().macboost_predict_contrib(handle.ptr, _f32(xf), rows, cols, _f32(out),
                                      ctypes.byref(err)) != 0:
        raise MacBoostError(_take_error(err))
    return out.reshape(rows, k * (cols + 1))


def feature_importance(handle: _Handle, importance_type: str = "gain") -> np.ndarray:
    out = np.empty(num_features(handle), dtype=np.float32)
    t = 1 if importance_type == "split" else 0
    if lib().macboost_feature_importance(handle.ptr, t, _f32(out)) != 0:
        raise MacBoostError("feature_importance failed")
    return out


def save(handle: _Handle, path) -> None:
    err = ctypes.c_char_p()
    if lib().macboost_save(handle.ptr, str(path).encode(), ctypes.byref(err)) != 0:
        raise MacBoostError(_take_error(err))


def load(path) -> _Handle:
    err = ctypes.c_char_p()
    ptr = lib().macboost_load(str(path).encode(), ctypes.byref(err))
    if not ptr:
        raise MacBoostError(_take_error(err))
    return _Handle(ptr)


def num_trees(handle):
    return int(lib().macboost_num_trees(handle.ptr))


def num_features(handle):
    return int(lib().macboost_num_features(handle.ptr))


def num_classes(handle):
    return int(lib().macboost_num_classes(handle.ptr))


def best_iteration(handle):
    return int(lib().macboost_best_iteration(handle.ptr))


def warnings(handle) -> list[str]:
    p = lib().macboost_warnings(handle.ptr)
    if not p:
        return []
    s = ctypes.cast(p, ctypes.c_char_p).value.decode()
    lib().macboost_free_string(p)
    return s.split("\n")


def eval_history(handle) -> np.ndarray:
    """The validation metric after every boosting round of the fit."""
    n = int(lib().mbx_eval_history(handle.ptr, None, 0))
    out = np.empty(max(n, 0), np.float32)
    if n > 0:
        lib().mbx_eval_history(handle.ptr, out.ctypes.data, n)
    return out


def version() -> str:
    return lib().mbx_version().decode()


def friedman(rows: int, cols: int, seed: int, noise: float = 1.0):
    """Friedman #1 data (DataGen.friedman): feature-major X [cols, rows] and y."""
    if cols < 5:
        raise ValueError("friedman needs cols >= 5 (DataGen.swift:69)")
    x = np.empty((cols, rows), dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib().mbx_friedman(rows, cols, ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), noise,
                       x.ctypes.data, y.ctypes.data)
    return x, y


def profile_train(enable: bool = True, every: int = 1) -> None:
    """HIP-event timing of the histogram launches of every every-th tree of
    each later train() call in this process (enable=False stops it)."""
    err = ctypes.c_char_p()
    if lib().mbx_profile_global(max(1, every) if enable else 0, ctypes.byref(err)) != 0:
        raise MacBoostError(_take_error(err))


def train_hist_stats(levels: int = 16):
    """(launches, ms, algorithmic bytes, built rows per level, ms per level) of
    the histogram kernel over the train() calls timed since profile_train()."""
    n, ms, b = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double()
    built = np.zeros(levels, np.int64)
    lms = np.zeros(levels, np.float64)
    err = ctypes.c_char_p()
    if lib().mbx_profile_global_stats(levels, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(b),
                                      built.ctypes.data, lms.ctypes.data,
                                      ctypes.byref(err)) != 0:
        raise MacBoostError(_take_error(err))
    return int(n.value), float(ms.value), float(b.value), built, lms


class Trainer:
    """Incremental trainer (mbx_trainer_*): bins once, grows trees on demand."""

    def __init__(self, config: dict, X, y, eval_set=None, sample_weight=None,
                 feature_major=False):
        cfg, xf, rows, cols, rm, yv, w, xv, vrows, yvv = _prep_train(
            config, X, y, eval_set, sample_weight, feature_major)
        err = ctypes.c_char_p()
        self.ptr = lib().mbx_trainer_create(cfg, _f32(xf), rows, cols, rm, _f32(yv), _f32(w),
                                            _f32(xv), vrows, _f32(yvv), ctypes.byref(err))
        if not self.ptr:
            raise MacBoostError(_take_error(err))
        self.rows, self.cols = rows, cols

    def grow(self, n: int) -> None:
        err = ctypes.c_char_p()
        if lib().mbx_trainer_grow(self.ptr, n, ctypes.byref(err)) != 0:
            raise MacBoostError(_take_error(err))

    def call(self, name: str, *args) -> None:
        """One mbk_* entry point on this context (the error argument is added)."""
        err = ctypes.c_char_p()
        self._check(getattr(lib(), name)(self.ptr, *args, ctypes.byref(err)), err)

    def profile(self, enable: bool = True) -> None:
        err = ctypes.c_char_p()
        lib().mbx_trainer_profile(self.ptr, 1 if enable else 0, ctypes.byref(err))

    def hist_stats(self):
        n = ctypes.c_int64()
        ms = ctypes.c_double()
        b = ctypes.c_double()
        err = ctypes.c_char_p()
        if lib().mbx_trainer_hist_stats(self.ptr, ctypes.byref(n), ctypes.byref(ms),
                                        ctypes.byref(b), ctypes.byref(err)) != 0:
            raise MacBoostError(_take_error(err))
        return int(n.value), float(ms.value), float(b.value)

    def level_stats(self, levels: int):
        """Per-level (built rows, live rows, histogram ms) summed over the
        profiled trees."""
        built = np.zeros(levels, np.int64)
        active = np.zeros(levels, np.int64)
        ms = np.zeros(levels, np.float64)
        err = ctypes.c_char_p()
        if lib().mbx_trainer_level_stats(self.ptr, levels, built.ctypes.data, active.ctypes.data,
                                         ms.ctypes.data, ctypes.byref(err)) != 0:
            raise MacBoostError(_take_error(err))
        return built, active, ms

    def setup_seconds(self):
        e = ctypes.c_double()
        b = ctypes.c_double()
        lib().mbx_trainer_setup_seconds(self.ptr, ctypes.byref(e), ctypes.byref(b))
        return float(e.value), float(b.value)

    def booster(self) -> _Handle:
        err = ctypes.c_char_p()
        ptr = lib().mbx_trainer_booster(self.ptr, ctypes.byref(err))
        if not ptr:
            raise MacBoostError(_take_error(err))
        return _Handle(ptr)

    def close(self):
        if getattr(self, "ptr", None) and _lib_instance is not None:
            _lib_instance.mbx_trainer_free(self.ptr)
            self.ptr = None

    def __del__(self):
        self.close()


class Context:
    """Kernel seam (mbk_*): one device, one stream, device buffers."""

    def __init__(self, device: int = 0):
        self.ptr = _P()
        err = ctypes.c_char_p()
        if lib().mbk_context_create(device, ctypes.byref(self.ptr), ctypes.byref(err)) != 0:
            raise MacBoostError(_take_error(err))
        self._bufs = []

    def _check(self, rc, err):
        if rc != 0:
            raise MacBoostError(_take_error(err))

    def alloc(self, nbytes: int) -> int:
        p = _P()
        err = ctypes.c_char_p()
        self._check(lib().mbk_device_alloc(self.ptr, nbytes, ctypes.byref(p), ctypes.byref(err)),
                    err)
        self._bufs.append(p.value)
        return p.value

    def upload(self, arr: np.ndarray) -> int:
        a = np.ascontiguousarray(arr)
        d = self.alloc(a.nbytes)
        err = ctypes.c_char_p()
        self._check(lib().mbk_copy_to_device(self.ptr, d, a.ctypes.data, a.nbytes,
                                             ctypes.byref(err)), err)
        return d

    def download(self, dptr: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        err = ctypes.c_char_p()
        self._check(lib().mbk_copy_to_host(self.ptr, out.ctypes.data, dptr, out.nbytes,
                                           ctypes.byref(err)), err)
        return out

    def fit(self, config: dict, x_dev: int, rows: int, cols: int, y, row_major=False,
            sample_weight=None, eval_set=None) -> _Handle:
        """mbk_fit: a whole fit over raw features already in device memory
        (x_dev, [cols][rows] or with row_major [rows][cols] float32)."""
        yv = _column(y, rows, "y")
        w = None if sample_weight is None else _column(sample_weight, rows, "sample_weight")
        xv, yvv, vrows = _eval_arrays(eval_set, cols)
        err = ctypes.c_char_p()
        ptr = lib().mbk_fit(self.ptr, json.dumps(config).encode(), x_dev, rows, cols,
                            1 if row_major else 0, _f32(yv), _f32(w), _f32(xv), vrows,
                            _f32(yvv), ctypes.byref(err))
        if not ptr:
            raise MacBoostError(_take_error(err))
        return _Handle(ptr)

    def call(self, name: str, *args) -> None:
        """One mbk_* entry point on this context (the error argument is added)."""
        err = ctypes.c_char_p()
        self._check(getattr(lib(), name)(self.ptr, *args, ctypes.byref(err)), err)

    def profile(self, enable: bool = True, every: int = 1) -> None:
        """HIP-event timing of the histogram launches of every every-th tree
        of later fits (enable=False stops it)."""
        err = ctypes.c_char_p()
        self._check(lib().mbx_context_profile(self.ptr, max(1, every) if enable else 0,
                                              ctypes.byref(err)), err)

    def hist_stats(self, levels: int = 16):
        """(launches, ms, algorithmic bytes, built rows per level, ms per level)
        of the histogram kernel over the profiled fits."""
        n, ms, b = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double()
        built = np.zeros(levels, np.int64)
        lms = np.zeros(levels, np.float64)
        err = ctypes.c_char_p()
        self._check(lib().mbx_context_hist_stats(self.ptr, levels, ctypes.byref(n),
                                                 ctypes.byref(ms), ctypes.byref(b),
                                                 built.ctypes.data, lms.ctypes.data,
                                                 ctypes.byref(err)), err)
        return int(n.value), float(ms.value), float(b.value), built, lms

    def sync(self):
        err = ctypes.c_char_p()
        self._check(lib().mbk_synchronize(self.ptr, ctypes.byref(err)), err)

    def close(self):
        if getattr(self, "ptr", None) and self.ptr.value and _lib_instance is not None:
            for b in self._bufs:
                _lib_instance.mbk_device_free(self.ptr, b)
            self._bufs = []
            _lib_instance.mbk_context_destroy(self.ptr)
            self.ptr = _P()

    def __del__(self):
        self.close()


class Dataset:
    """A preprocessed training set (the reference's BinnedDataset,
    Dataset.swift:11-86): quantile-binned features in the .mbds tile-8 layout,
    edges, labels, bin count, categorical layout and feature names.  Build it
    with Dataset.make (edges and bins on the GPU), or Dataset.load a .mbds
    file; train_dataset fits from it without binning again."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    @classmethod
    def make(cls, config: dict, X, y, feature_names=None, feature_major=False) -> "Dataset":
        xf = np.ascontiguousarray(_matrix(X))
        if feature_major:
            cols, rows = xf.shape
        else:
            rows, cols = xf.shape
        yv = _column(y, rows, "y")
        if feature_names is not None and len(feature_names) != cols:
            raise ValueError(f"feature_names has {len(feature_names)} entries, X has {cols} "
                             "features")
        names = None if feature_names is None else json.dumps(list(feature_names)).encode()
        err = ctypes.c_char_p()
        ptr = lib().mbx_dataset_make(json.dumps(config).encode(), _f32(xf), rows, cols,
                                     0 if feature_major else 1, _f32(yv), names,
                                     ctypes.byref(err))
        if not ptr:
            raise MacBoostError(_take_error(err))
        return cls(ptr)

    @classmethod
    def load(cls, path) -> "Dataset":
        err = ctypes.c_char_p()
        ptr = lib().mbx_dataset_load(str(path).encode(), ctypes.byref(err))
        if not ptr:
            raise MacBoostError(_take_error(err))
        return cls(ptr)

    def save(self, path) -> None:
        err = ctypes.c_char_p()
        if lib().mbx_dataset_save(self.ptr, str(path).encode(), ctypes.byref(err)) != 0:
            raise MacBoostError(_take_error(err))

    def _info(self):
        r, c = ctypes.c_int64(), ctypes.c_int64()
        nb, nc = ctypes.c_int32(), ctypes.c_int32()
        lib().mbx_dataset_info(self.ptr, ctypes.byref(r), ctypes.byref(c), ctypes.byref(nb),
                               ctypes.byref(nc))
        return r.value, c.value, nb.value, nc.value

    @property
    def rows(self) -> int:
        return self._info()[0]

    @property
    def cols(self) -> int:
        return self._info()[1]

    @property
    def num_bins(self) -> int:
        return self._info()[2]

    def arrays(self):
        """(categorical, labels, edges [cols][num_bins-2], bins [ceil(cols/8)][rows][8])."""
        rows, cols, nb, nc = self._info()
        cat = np.empty(nc, np.int32)
        labels = np.empty(rows, np.float32)
        edges = np.empty((cols, max(nb - 2, 0)), np.float32)
        bins = np.empty(((cols + 7) // 8, rows, 8), np.uint8)
        lib().mbx_dataset_copy(self.ptr, cat.ctypes.data, labels.ctypes.data, edges.ctypes.data,
                               bins.ctypes.data)
        return cat, labels, edges, bins

    @property
    def feature_names(self):
        p = lib().mbx_dataset_feature_names(self.ptr)
        if not p:
            return None
        s = ctypes.cast(p, ctypes.c_char_p).value.decode()
        lib().macboost_free_string(ctypes.cast(p, ctypes.c_void_p))
        return json.loads(s)

    def close(self):
        if getattr(self, "ptr", None) and _lib_instance is not None:
            _lib_instance.mbx_dataset_free(self.ptr)
        self.ptr = None

    def __del__(self):
        self.close()


def train_dataset(config: dict, dataset: Dataset, eval_set=None, sample_weight=None) -> _Handle:
    """fit(dataset:) (Booster.swift:375-389): the dataset's bins, bin count,
    categorical layout and labels are used."""
    rows, cols = dataset.rows, dataset.cols
    w = None if sample_weight is None else _column(sample_weight, rows, "sample_weight")
    xv, yvv, vrows = _eval_arrays(eval_set, cols)
    err = ctypes.c_char_p()
    ptr = lib().mbx_dataset_train(json.dumps(config).encode(), dataset.ptr, _f32(w), _f32(xv),
                                  vrows, _f32(yvv), ctypes.byref(err))
    if not ptr:
        raise MacBoostError(_take_error(err))
    return _Handle(ptr)
