"""ctypes front end of the CPU oracle (oracle/liboracle.so).

Test infrastructure only: tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it to compare results.  Every function
mirrors one entry of ``oracle/mbo_oracle.h``.
"""
from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = ROOT / "oracle" / "liboracle.so"

# planted mistakes (oracle/mbo_oracle.h ORC_PLANT_*): tests only
PLANT_FIFO_PICK = 1
PLANT_GOSS_NO_SEED = 2
PLANT_EDGE_K = 3
PLANT_EDGE_K2 = 4
PLANT_EDGE_NUMBINS = 5
PLANT_EDGE_M1 = 6
PLANT_EDGE_CEIL = 7
PLANT_EDGE_NOSTRIDE = 8

FLAG_DEFAULT_LEFT = 1
FLAG_CATEGORICAL = 2
OBJ_L2, OBJ_LOGISTIC, OBJ_MAE, OBJ_HUBER, OBJ_QUANTILE, OBJ_POISSON, OBJ_TWEEDIE, OBJ_MULTICLASS = range(8)

_lib = None


def set_threads(n: int) -> None:
    """Threads of the oracle's parallel loops (<= 0: every processor).  Results
    are identical at any count."""
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _configure(_lib)
    return _lib


class OrcParams(ctypes.Structure):
    _fields_ = [
        ("num_trees", ctypes.c_int32), ("max_depth", ctypes.c_int32),
        ("num_bins", ctypes.c_int32), ("objective", ctypes.c_int32),
        ("num_leaves", ctypes.c_int32), ("learning_rate", ctypes.c_float),
        ("lambda_", ctypes.c_float), ("min_child_hess", ctypes.c_float),
        ("min_split_gain", ctypes.c_float), ("cat_smooth", ctypes.c_float),
        ("alpha", ctypes.c_float), ("aux", ctypes.c_float),
        ("goss", ctypes.c_int32), ("goss_top_rate", ctypes.c_float),
        ("goss_other_rate", ctypes.c_float), ("subsample", ctypes.c_float),
        ("num_classes", ctypes.c_int32), ("feature_fraction", ctypes.c_float),
        ("plant", ctypes.c_int32), ("allowed", ctypes.c_void_p),
    ]


class OrcSplit(ctypes.Structure):
    _fields_ = [
        ("gain", ctypes.c_float), ("bin", ctypes.c_uint32), ("gl", ctypes.c_float),
        ("hl", ctypes.c_float), ("flags", ctypes.c_uint32),
        ("gl_int", ctypes.c_int64), ("hl_int", ctypes.c_int64),
    ]


class OrcForest(ctypes.Structure):
    _fields_ = [
        ("num_trees", ctypes.c_int32), ("nodes_per_tree", ctypes.c_int32),
        ("feature", ctypes.c_void_p), ("threshold", ctypes.c_void_p),
        ("leaf", ctypes.c_void_p), ("flags", ctypes.c_void_p),
        ("cat_mask", ctypes.c_void_p), ("gain", ctypes.c_void_p),
        ("cover", ctypes.c_void_p), ("split_bin", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float


def _configure(l: ctypes.CDLL) -> None:
    l.orc_set_threads.restype = None
    l.orc_set_threads.argtypes = [ctypes.c_int32]
    l.orc_get_threads.restype = ctypes.c_int32
    l.orc_get_threads.argtypes = []
    l.orc_splitmix_next.restype = ctypes.c_uint64
    l.orc_splitmix_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    l.orc_friedman.argtypes = [_I64, _I32, ctypes.c_uint64, _F, _P, _P]
    l.orc_compute_edges.argtypes = [_P, _I64, _I32, _I64, _I64, _I32, _P, _I64, _P]
    l.orc_compute_edges_planted.argtypes = [_P, _I64, _I32, _I64, _I64, _I32, _P, _I64, _P,
                                            _I32]
    l.orc_bin_matrix.argtypes = [_P, _I64, _I32, _I64, _I64, _P, _P, _I32, _P]
    l.orc_base_score.restype = _F
    l.orc_base_score.argtypes = [_P, _P, _I64, _I32, _F]
    l.orc_label_quantile.restype = _F
    l.orc_label_quantile.argtypes = [_P, _I64, _F]
    l.orc_gradients_mc.restype = None
    l.orc_gradients_mc.argtypes = [_P, _P, _P, _I64, _I32, _I32, _P, _P, _P, _P]
    l.orc_base_scores_mc.restype = None
    l.orc_base_scores_mc.argtypes = [_P, _P, _I64, _I32, _P]
    l.orc_gradients.argtypes = [_P, _P, _P, _I64, _I32, _F, _F, _P, _P, _P, _P]
    l.orc_quantize.argtypes = [_P, _P, _I64, _F, _F, _P]
    l.orc_hist_node.argtypes = [_P, _I64, _I32, _I32, _P, _P, _I64, _P, _P]
    l.orc_find_split.argtypes = [_P, _P, _I32, ctypes.c_int, ctypes.c_int, _I64, _I64, _F,
                                 _F, _F, _F, _F, ctypes.POINTER(OrcSplit)]
    l.orc_cat_order.restype = _I32
    l.orc_cat_order.argtypes = [_P, _P, _I32, _F, _F, _F, _P]
    l.orc_fit.restype = ctypes.c_int
    l.orc_fit.argtypes = [ctypes.POINTER(OrcParams), _P, _I64, _I32, _P, _P, _P, _P, _P, _F,
                          _P, ctypes.POINTER(OrcForest)]
    l.orc_predict.argtypes = [ctypes.POINTER(OrcForest), _F, _I32, _P, _I64, _I32, _P]
    l.orc_treeshap.argtypes = [ctypes.POINTER(OrcForest), _F, _I32, _P, _I64, _I32, _P]
    l.orc_shap_bias.restype = ctypes.c_double
    l.orc_shap_bias.argtypes = [ctypes.POINTER(OrcForest), _F]


def _ptr(a):
    return None if a is None else a.ctypes.data


# --------------------------------------------------------------------------
# data generation / binning
# --------------------------------------------------------------------------

def splitmix_stream(seed: int, n: int) -> np.ndarray:
    s = ctypes.c_uint64(seed)
    return np.array([lib().orc_splitmix_next(ctypes.byref(s)) for _ in range(n)], dtype=np.uint64)


def friedman(rows: int, cols: int, seed: int, noise: float = 1.0):
    """Feature-major X [cols, rows] and y, DataGen.friedman."""
    if cols < 5:
        raise ValueError("friedman needs cols >= 5 (DataGen.swift:69)")
    x = np.empty((cols, rows), dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib().orc_friedman(rows, cols, ctypes.c_uint64(seed), noise, _ptr(x), _ptr(y))
    return x, y


def compute_edges(x_fm: np.ndarray, num_bins: int, is_cat=None, sample_cap: int = 200_000,
                  plant: int = 0, row_major: bool = False):
    """Quantile edges of a feature-major [cols, rows] matrix; row_major reads the
    transposed copy through the row/column strides instead. plant != 0 (tests only)
    plants one of the PLANT_EDGE_* mistakes."""
    cols, rows = x_fm.shape
    if row_major:
        x = np.ascontiguousarray(np.asarray(x_fm, dtype=np.float32).T)
        rs, cs = cols, 1
    else:
        x = np.ascontiguousarray(x_fm, dtype=np.float32)
        rs, cs = 1, rows
    cat = None if is_cat is None else np.ascontiguousarray(is_cat, dtype=np.uint8)
    edges = np.zeros((cols, num_bins - 2), dtype=np.float32)
    if plant:
        lib().orc_compute_edges_planted(_ptr(x), rows, cols, rs, cs, num_bins, _ptr(cat),
                                        sample_cap, _ptr(edges), plant)
    else:
        lib().orc_compute_edges(_ptr(x), rows, cols, rs, cs, num_bins, _ptr(cat), sample_cap,
                                _ptr(edges))
    return edges


def bin_matrix(x_fm: np.ndarray, edges: np.ndarray, num_bins: int, is_cat=None):
    cols, rows = x_fm.shape
    x_fm = np.ascontiguousarray(x_fm, dtype=np.float32)
    cat = None if is_cat is None else np.ascontiguousarray(is_cat, dtype=np.uint8)
    out = np.empty((cols, rows), dtype=np.uint8)
    lib().orc_bin_matrix(_ptr(x_fm), rows, cols, 1, rows, _ptr(edges), _ptr(cat), num_bins,
                         _ptr(out))
    return out


# --------------------------------------------------------------------------
# gradients / histograms / splits
# --------------------------------------------------------------------------

def base_score(y, w=None, objective=OBJ_L2, scale_pos_weight=1.0, alpha=0.9) -> float:
    y = np.ascontiguousarray(y, dtype=np.float32)
    w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    if objective in (OBJ_MAE, OBJ_QUANTILE):
        q = 0.5 if objective == OBJ_MAE else alpha
        return float(lib().orc_label_quantile(_ptr(y), len(y), q))
    return float(lib().orc_base_score(_ptr(y), _ptr(w), len(y), objective, scale_pos_weight))


def gradients(preds, y, w=None, objective=OBJ_L2, alpha=0.9, aux=1.0):
    n = len(y)
    preds = np.ascontiguousarray(preds, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    g = np.empty(n, np.float32)
    h = np.empty(n, np.float32)
    mg = np.zeros(1, np.float32)
    mh = np.zeros(1, np.float32)
    lib().orc_gradients(_ptr(preds), _ptr(y), _ptr(w), n, objective, alpha, aux, _ptr(g),
                        _ptr(h), _ptr(mg), _ptr(mh))
    return g, h, float(mg[0]), float(mh[0])


def quantize(g, h, max_g, max_h):
    out = np.empty(len(g), np.uint32)
    lib().orc_quantize(_ptr(np.ascontiguousarray(g, np.float32)),
                       _ptr(np.ascontiguousarray(h, np.float32)), len(g), max_g, max_h,
                       _ptr(out))
    return out


def hist_node(bins_fm, num_bins, ghq, rows_idx=None):
    cols, rows = bins_fm.shape
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    ghq = np.ascontiguousarray(ghq, np.uint32)
    idx = None if rows_idx is None else np.ascontiguousarray(rows_idx, np.uint32)
    n = rows if idx is None else len(idx)
    hg = np.empty((cols, num_bins), np.int64)
    hh = np.empty((cols, num_bins), np.int64)
    lib().orc_hist_node(_ptr(bins_fm), rows, cols, num_bins, _ptr(ghq), _ptr(idx), n, _ptr(hg),
                        _ptr(hh))
    return hg, hh


def find_split(hg, hh, is_cat, monotone, g_tot, h_tot, g_inv, h_inv, lam=1.0, mch=1.0,
               cat_smooth=10.0) -> OrcSplit:
    hg = np.ascontiguousarray(hg, np.int64)
    hh = np.ascontiguousarray(hh, np.int64)
    r = OrcSplit()
    lib().orc_find_split(_ptr(hg), _ptr(hh), len(hg), int(is_cat), int(monotone), int(g_tot),
                         int(h_tot), g_inv, h_inv, lam, mch, cat_smooth, ctypes.byref(r))
    return r


def cat_order(hg, hh, g_inv, h_inv, cat_smooth=10.0):
    hg = np.ascontiguousarray(hg, np.int64)
    hh = np.ascontiguousarray(hh, np.int64)
    order = np.zeros(256, np.uint16)
    m = lib().orc_cat_order(_ptr(hg), _ptr(hh), len(hg), g_inv, h_inv, cat_smooth, _ptr(order))
    return order[:m]


# --------------------------------------------------------------------------
# models
# --------------------------------------------------------------------------

@dataclass
class Forest:
    """Flat heap forest, [num_trees, nodes_per_tree] per array."""
    feature: np.ndarray
    threshold: np.ndarray
    leaf: np.ndarray
    flags: np.ndarray
    cat_mask: np.ndarray | None
    gain: np.ndarray
    cover: np.ndarray
    split_bin: np.ndarray | None = None

    @property
    def num_trees(self):
        return self.feature.shape[0]

    @property
    def nodes_per_tree(self):
        return self.feature.shape[1]

    @classmethod
    def empty(cls, num_trees, nodes, with_cats=True):
        return cls(
            feature=np.full((num_trees, nodes), -1, np.int32),
            threshold=np.zeros((num_trees, nodes), np.float32),
            leaf=np.zeros((num_trees, nodes), np.float32),
            flags=np.zeros((num_trees, nodes), np.uint8),
            cat_mask=np.zeros((num_trees, nodes, 8), np.uint32) if with_cats else None,
            gain=np.zeros((num_trees, nodes), np.float32),
            cover=np.zeros((num_trees, nodes), np.float32),
            split_bin=np.zeros((num_trees, nodes), np.uint32),
        )

    def c(self) -> OrcForest:
        for name in ("feature", "threshold", "leaf", "flags", "gain", "cover"):
            assert getattr(self, name).flags.c_contiguous
        f = OrcForest()
        f.num_trees = self.num_trees
        f.nodes_per_tree = self.nodes_per_tree
        f.feature = _ptr(self.feature)
        f.threshold = _ptr(self.threshold)
        f.leaf = _ptr(self.leaf)
        f.flags = _ptr(self.flags)
        f.cat_mask = _ptr(self.cat_mask)
        f.gain = _ptr(self.gain)
        f.cover = _ptr(self.cover)
        f.split_bin = _ptr(self.split_bin)
        return f


@dataclass
class OracleModel:
    forest: Forest
    base_score: float
    num_bins: int
    preds: np.ndarray             # [rows], or [K, rows] for multiclass
    edges: np.ndarray
    base_scores: list = None      # per class (multiclass)
    num_classes: int = 1


def base_scores_mc(y, w, num_classes):
    y = np.ascontiguousarray(y, np.float32)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    out = np.empty(num_classes, np.float32)
    lib().orc_base_scores_mc(_ptr(y), _ptr(w), len(y), num_classes, _ptr(out))
    return out


def gradients_mc(preds_kr, y, num_classes, cls, w=None):
    preds_kr = np.ascontiguousarray(preds_kr, np.float32)
    rows = preds_kr.shape[1]
    y = np.ascontiguousarray(y, np.float32)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    g = np.empty(rows, np.float32)
    h = np.empty(rows, np.float32)
    mg = np.zeros(1, np.float32)
    mh = np.zeros(1, np.float32)
    lib().orc_gradients_mc(_ptr(preds_kr), _ptr(y), _ptr(w), rows, num_classes, cls, _ptr(g),
                           _ptr(h), _ptr(mg), _ptr(mh))
    return g, h, float(mg[0]), float(mh[0])


def fit(bins_fm, y, *, edges, num_trees=100, max_depth=6, num_bins=256, objective=OBJ_L2,
        num_leaves=0, learning_rate=0.1, lam=1.0, min_child_hess=1.0, min_split_gain=0.0,
        cat_smooth=10.0, alpha=0.9, aux=1.0, w=None, is_cat=None, monotone=None,
        base=None, goss=False, goss_top_rate=0.2, goss_other_rate=0.1,
        subsample=1.0, num_classes=1, init_preds=None, feature_fraction=1.0,
        allowed_features=None, plant=0) -> OracleModel:
    cols, rows = bins_fm.shape
    K = num_classes if objective == OBJ_MULTICLASS else 1
    allowed = None
    if allowed_features is not None:
        allowed = np.zeros(cols, np.uint8)
        allowed[list(allowed_features)] = 1
    p = OrcParams(num_trees, max_depth, num_bins, objective, num_leaves, learning_rate, lam,
                  min_child_hess, min_split_gain, cat_smooth, alpha, aux, int(goss),
                  goss_top_rate, goss_other_rate, subsample, K, feature_fraction, plant,
                  None if allowed is None else allowed.ctypes.data)
    y = np.ascontiguousarray(y, np.float32)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    bases = None
    if K > 1:
        bases = base_scores_mc(y, w, K)
        base = 0.0
        preds = np.ascontiguousarray(np.repeat(bases[:, None], rows, axis=1))
    else:
        if base is None:
            base = base_score(y, w, objective, aux if objective == OBJ_LOGISTIC else 1.0, alpha)
        preds = np.full(rows, base, np.float32)
    if init_preds is not None:
        # warm start: running predictions begin at the init model's raw
        # scores (Booster.swift:849-866)
        preds = np.ascontiguousarray(np.array(init_preds, np.float32).reshape(preds.shape))
    nodes = (1 << (max_depth + 1)) - 1
    forest = Forest.empty(num_trees * K, nodes)
    cat = None if is_cat is None else np.ascontiguousarray(is_cat, np.uint8)
    mono = None if monotone is None else np.ascontiguousarray(monotone, np.int8)
    edges = np.ascontiguousarray(edges, np.float32)
    fc = forest.c()
    rc = lib().orc_fit(ctypes.byref(p), _ptr(np.ascontiguousarray(bins_fm, np.uint8)), rows,
                       cols, _ptr(y), _ptr(w), _ptr(cat), _ptr(mono), _ptr(edges), base,
                       _ptr(preds), ctypes.byref(fc))
    if rc != 0:
        raise RuntimeError(f"orc_fit failed: {rc}")
    return OracleModel(forest, float(base), num_bins, preds, edges,
                       None if bases is None else [float(b) for b in bases], K)


def class_forest(forest: Forest, k: int, num_classes: int) -> Forest:
    """The trees of class k (tree t fits class t % K), in order."""
    def sel(a):
        return None if a is None else np.ascontiguousarray(a[k::num_classes])
    return Forest(sel(forest.feature), sel(forest.threshold), sel(forest.leaf), sel(forest.flags),
                  sel(forest.cat_mask), sel(forest.gain), sel(forest.cover), sel(forest.split_bin))


def predict_mc(forest: Forest, base_scores, num_bins: int, x_fm) -> np.ndarray:
    """Multiclass raw scores [rows, K]: class k sums its own trees in order
    from its base score (predict_forest, Shaders.swift:1548-1578)."""
    K = len(base_scores)
    return np.stack([predict(class_forest(forest, k, K), base_scores[k], num_bins, x_fm)
                     for k in range(K)], axis=1)


def treeshap_mc(forest: Forest, base_scores, num_bins: int, x_fm) -> np.ndarray:
    """Multiclass contributions [rows, K * (cols + 1)], one block per class."""
    K = len(base_scores)
    return np.concatenate([treeshap(class_forest(forest, k, K), base_scores[k], num_bins, x_fm)
                           for k in range(K)], axis=1)


def predict(forest: Forest, base: float, num_bins: int, x_fm) -> np.ndarray:
    cols, rows = x_fm.shape
    out = np.empty(rows, np.float32)
    fc = forest.c()
    lib().orc_predict(ctypes.byref(fc), base, num_bins - 1,
                      _ptr(np.ascontiguousarray(x_fm, np.float32)), rows, cols, _ptr(out))
    return out


def treeshap(forest: Forest, base: float, num_bins: int, x_fm) -> np.ndarray:
    cols, rows = x_fm.shape
    out = np.empty((rows, cols + 1), np.float32)
    fc = forest.c()
    lib().orc_treeshap(ctypes.byref(fc), base, num_bins - 1,
                       _ptr(np.ascontiguousarray(x_fm, np.float32)), rows, cols, _ptr(out))
    return out


def shap_bias(forest: Forest, base: float) -> float:
    fc = forest.c()
    return float(lib().orc_shap_bias(ctypes.byref(fc), base))


def sample_rows(g, h, max_g, tree, *, learning_rate=0.1, goss=False, goss_top_rate=0.2,
                goss_other_rate=0.1, subsample=1.0, plant=0):
    """orc_sample_rows: (kept mask, amplified g, amplified h, wmax_g, wmax_h),
    or None when the tree does not sample."""
    p = OrcParams(1, 6, 256, OBJ_L2, 0, learning_rate, 1.0, 1.0, 0.0, 10.0, 0.9, 1.0,
                  int(goss), goss_top_rate, goss_other_rate, subsample, 1, 1.0, plant, None)
    l = lib()
    l.orc_sampling_active.restype = ctypes.c_int
    l.orc_sampling_active.argtypes = [ctypes.c_void_p, ctypes.c_int32]
    if not l.orc_sampling_active(ctypes.byref(p), tree):
        return None
    g = np.array(g, np.float32)
    h = np.array(h, np.float32)
    kept = np.zeros(len(g), np.uint8)
    wg = np.zeros(1, np.float32)
    wh = np.zeros(1, np.float32)
    l.orc_sample_rows.restype = ctypes.c_int64
    l.orc_sample_rows.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                  ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    n = l.orc_sample_rows(ctypes.byref(p), tree, _ptr(g), _ptr(h), len(g), max_g, _ptr(kept),
                          _ptr(wg), _ptr(wh))
    assert n == int(kept.sum())
    return kept.astype(bool), g, h, float(wg[0]), float(wh[0])


def fit_raw(x_fm, y, num_bins=256, is_cat=None, **kw) -> OracleModel:
    """Edges + binning + fit, the whole reference fit path on raw features."""
    edges = compute_edges(x_fm, num_bins, is_cat)
    bins = bin_matrix(x_fm, edges, num_bins, is_cat)
    return fit(bins, y, edges=edges, num_bins=num_bins, is_cat=is_cat, **kw)




class SplitMix:
    """SplitMix64 stream (DataGen.swift:6-26) driven through the oracle."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)
        l = lib()
        l.orc_splitmix_uniform.restype = ctypes.c_float
        l.orc_splitmix_uniform.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        l.orc_splitmix_normal.restype = ctypes.c_float
        l.orc_splitmix_normal.argtypes = [ctypes.POINTER(ctypes.c_uint64)]

    def next(self) -> int:
        return int(lib().orc_splitmix_next(ctypes.byref(self.state)))

    def uniform(self) -> float:
        return lib().orc_splitmix_uniform(ctypes.byref(self.state))

    def normal(self) -> float:
        return lib().orc_splitmix_normal(ctypes.byref(self.state))

    def uniforms(self, n: int) -> np.ndarray:
        return np.array([self.uniform() for _ in range(n)], dtype=np.float32)


# --------------------------------------------------------------------------
# Boruta feature selection (FeatureSelection.swift:45-190)
# --------------------------------------------------------------------------

def shadow_bins(bins_fm, half_bits, seed):
    l = lib()
    l.orc_shadow_bins.restype = None
    l.orc_shadow_bins.argtypes = [_P, _I64, _I32, ctypes.c_uint32, ctypes.c_uint32, _P]
    cols, rows = bins_fm.shape
    src = np.ascontiguousarray(bins_fm, np.uint8)
    out = np.empty((2 * cols, rows), np.uint8)
    l.orc_shadow_bins(_ptr(src), rows, cols, half_bits, seed & 0xFFFFFFFF, _ptr(out))
    return out


def shadow_perm(i, n, half_bits, seed):
    l = lib()
    l.orc_shadow_perm.restype = ctypes.c_uint32
    l.orc_shadow_perm.argtypes = [ctypes.c_uint32] * 4
    return int(l.orc_shadow_perm(i, n, half_bits, seed & 0xFFFFFFFF))


def gain_importance(forest: Forest, num_features: int) -> np.ndarray:
    """featureImportance(type: .gain) (Booster.swift:1926-1940): per tree a
    stack walk from the root, f32 sums in that visiting order."""
    imp = np.zeros(num_features, np.float32)
    for t in range(forest.num_trees):
        stack = [0]
        while stack:
            n = stack.pop()
            f = int(forest.feature[t, n])
            if f < 0:
                continue
            imp[f] = np.float32(imp[f] + forest.gain[t, n])
            stack.append(2 * n + 1)
            stack.append(2 * n + 2)
    return imp


def binomial_tail(k, rounds):
    """P[Binomial(rounds, 0.5) >= k], accumulated as FeatureSelection.swift:193-203."""
    if k <= 0:
        return 1.0
    pmf = 0.5 ** rounds
    tail = 0.0
    for i in range(rounds + 1):
        if i >= k:
            tail += pmf
        if i < rounds:
            pmf *= (rounds - i) / (i + 1)
    return min(1.0, tail)


def select_features(x_fm, y, *, rounds=20, trees=None, alpha=0.05, seed=0, num_bins=256,
                    is_cat=None, num_trees=100, **fit_kw):
    """Boruta: bins once, then per round a fit on [bins | shadow(bins)] and a
    vote of each real feature's gain against the best shadow's.  Returns
    (hits, decision 2/1/0, gain ratio)."""
    cols, rows = x_fm.shape
    edges = compute_edges(x_fm, num_bins, is_cat)
    bins = bin_matrix(x_fm, edges, num_bins, is_cat)
    edges2 = np.ascontiguousarray(np.vstack([edges, edges]))
    cat2 = None if is_cat is None else np.concatenate([is_cat, is_cat]).astype(np.uint8)
    bits = 1
    while (1 << bits) < rows:
        bits += 1
    half = (bits + 1) // 2
    n_trees = trees if trees is not None else min(num_trees, 100)
    hits = np.zeros(cols, np.int64)
    gain_sum = np.zeros(cols, np.float64)
    shadow_sum = 0.0
    for r in range(rounds):
        rseed = (seed + r * 0x9E3779B97F4A7C15 + 1) & 0xFFFFFFFF
        b2 = shadow_bins(bins, half, rseed)
        m = fit(b2, y, edges=edges2, num_bins=num_bins, is_cat=cat2, num_trees=n_trees, **fit_kw)
        g = gain_importance(m.forest, 2 * cols)
        mx = g[cols:].max()
        hits += g[:cols] > mx
        gain_sum += g[:cols].astype(np.float64)
        shadow_sum += float(mx)
    cutoff = alpha / cols
    dec = np.ones(cols, np.int32)
    for f in range(cols):
        if binomial_tail(int(hits[f]), rounds) < cutoff:
            dec[f] = 2
        elif binomial_tail(rounds - int(hits[f]), rounds) < cutoff:
            dec[f] = 0
    ratio = (gain_sum / max(shadow_sum, np.finfo(np.float64).tiny)).astype(np.float32)
    return hits.astype(np.int32), dec, ratio
