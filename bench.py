#!/usr/bin/env python3
"""Benchmark of the MI355X tree-build path.

Workload (the headline metric): Friedman #1 regression, 10M rows x 100 fp32
features, 256 bins, level-wise depth 6, lr 0.1, L2.  A step is one boosting
iteration (one depth-6 tree) over the binned matrix resident in HBM.  W
untimed warm-up trees, then K timed trees; value = K / seconds (trees/s).

Also reported: the histogram kernel's roofline (algorithmic bytes = sum over
built nodes of rows*(features+4), timed with HIP events on the kernel's own
stream), the end-to-end fit time including edges/upload/binning, and the CPU
oracle timed on this host (single thread) on a bounded sample of the same
workload.  Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
REFERENCE_TREES_PER_S = 25.6      # 100 trees in 3.9 s on an M4 Max (README.md:73)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(x, y, rows, cols, trees):
    """The oracle (single-threaded C) on the first `rows` rows, `trees` trees."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    xs = np.ascontiguousarray(x[:, :rows])
    ys = np.ascontiguousarray(y[:rows])
    t0 = time.perf_counter()
    edges = O.compute_edges(xs, 256)
    bins = O.bin_matrix(xs, edges, 256)
    t_bin = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.fit(bins, ys, edges=edges, num_trees=trees, max_depth=6, num_bins=256)
    t_fit = time.perf_counter() - t0
    return t_bin, t_fit


def measure_extras(mb, x, y, cols, trees, with_cpu):
    """Leaf-wise growth (63 leaves, depth 6) on the same 10M rows, then batch
    predict of 500k held-out rows and TreeSHAP of 200k rows with that model.
    Predict is checked bit for bit and TreeSHAP to 1e-5 relative against the
    oracle on row samples."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    import model_io
    out = {}
    params = {"num_trees": trees + 2, "max_depth": 6, "num_bins": 256, "learning_rate": 0.1,
              "num_leaves": 63}
    tr = mb.Trainer(params, x, y, feature_major=True)
    tr.grow(2)
    t0 = time.perf_counter()
    tr.grow(trees)
    el = time.perf_counter() - t0
    h = tr.booster()
    tr.close()
    out["leafwise"] = {"workload": "friedman1 10M x 100, 63 leaves, depth 6, 256 bins",
                       "trees": trees, "seconds": el, "trees_per_s": trees / el}
    log(f"leaf-wise: {trees} trees in {el:.3f}s = {trees / el:.1f} trees/s")
    obj = model_io.saved_model(h)
    forest = model_io.forest_from_json(obj)
    base, nb = obj["baseScore"], obj["numBins"]
    xp, _ = mb.friedman(500_000, cols, 42 + 999)
    mb.predict(h, xp[:, :1000], feature_major=True)
    t0 = time.perf_counter()
    pp = mb.predict(h, xp, feature_major=True)
    el = time.perf_counter() - t0
    sample = np.ascontiguousarray(xp[:, :20_000])
    t1 = time.perf_counter()
    want = O.predict(forest, base, nb, sample)
    cpu_el = time.perf_counter() - t1
    exact = bool(np.array_equal(pp[:20_000], want))
    out["predict"] = {"rows": 500_000, "trees": int(forest.num_trees), "seconds": el,
                      "rows_per_s": 500_000 / el, "bit_exact_vs_oracle_20k_rows": exact,
                      "note": "through macboost_predict: host X copied to HBM and back",
                      "cpu_oracle_rows_per_s_1_core": 20_000 / cpu_el}
    log(f"predict 500k x {forest.num_trees} trees: {el * 1e3:.1f} ms, bit-exact={exact}")
    xs = np.ascontiguousarray(xp[:, :200_000])
    mb.predict_contrib(h, xs[:, :1000], feature_major=True)
    t0 = time.perf_counter()
    c = mb.predict_contrib(h, xs, feature_major=True)
    el = time.perf_counter() - t0
    n_chk = 500
    t1 = time.perf_counter()
    ref = O.treeshap(forest, base, nb, np.ascontiguousarray(xs[:, :n_chk]))
    cpu_el = time.perf_counter() - t1
    ok = bool(np.allclose(c[:n_chk], ref, rtol=1e-5, atol=1e-6))
    out["treeshap"] = {"rows": 200_000, "trees": int(forest.num_trees), "seconds": el,
                       "row_trees_per_s": 200_000 * forest.num_trees / el,
                       "within_1e-5_rel_vs_oracle_500_rows": ok,
                       "cpu_oracle_row_trees_per_s_1_core": n_chk * forest.num_trees / cpu_el}
    log(f"TreeSHAP 200k x {forest.num_trees} trees: {el * 1e3:.1f} ms, within tol={ok}")
    del h
    out.update(measure_configs(mb, trees))
    return out


def measure_configs(mb, trees):
    """Whole fits through macboost_train (upload, device edges and binning,
    trees) on the NaN + categorical and HIGGS-like workloads."""
    import datasets as D
    out = {}
    x, y, cats = D.c3_mixed(1_000_000, 42)
    xv, yv, _ = D.c3_mixed(200_000, 42 + 999)
    params = {"num_trees": trees, "max_depth": 6, "num_bins": 256, "categorical_features": cats}
    mb.train(dict(params, num_trees=2), x[:, :100_000], y[:100_000], feature_major=True)
    t0 = time.perf_counter()
    h = mb.train(params, x, y, eval_set=(xv.T, yv), feature_major=True)
    el = time.perf_counter() - t0
    pv = mb.predict(h, xv, feature_major=True)
    rmse = float(np.sqrt(np.mean((pv.astype(np.float64) - yv) ** 2)))
    out["nan_categorical_1m"] = {
        "workload": "friedman1 1M x 100, 20 categorical columns (cardinality 2..64), 20% NaN, "
                    "200k validation rows evaluated after every tree",
        "trees": trees, "fit_seconds": el, "valid_rmse": rmse,
        "note": "whole macboost_train call: upload, device edges and binning, trees, readback"}
    log(f"NaN+categorical 1M: {trees} trees in {el:.3f}s, valid RMSE {rmse:.4f}")
    del h, x, xv
    x, y = D.c4_higgs_like(10_500_000, 42)
    n = 10_000_000
    xtr, ytr = np.ascontiguousarray(x[:, :n]), y[:n]
    xte, yte = np.ascontiguousarray(x[:, n:]), y[n:]
    del x
    params = {"num_trees": trees, "max_depth": 6, "num_bins": 256, "objective": "binary"}
    t0 = time.perf_counter()
    h = mb.train(params, xtr, ytr, feature_major=True)
    el = time.perf_counter() - t0
    p = mb.predict(h, xte, feature_major=True)
    from sklearn.metrics import roc_auc_score
    auc = float(roc_auc_score(yte, p))
    out["higgs_like_10m"] = {
        "workload": "HIGGS-like 10M x 28 (synthetic), logistic, 500k held out",
        "trees": trees, "fit_seconds": el, "auc": auc,
        "note": "whole macboost_train call; synthetic stand-in for HIGGS, so the "
                "reference's 2.8 s / AUC 0.8128 on real HIGGS is not comparable"}
    log(f"HIGGS-like 10M: {trees} trees in {el:.3f}s, AUC {auc:.4f}")
    del h
    params["goss"] = True                            # GOSS(0.2, 0.1)
    t0 = time.perf_counter()
    h = mb.train(params, xtr, ytr, feature_major=True)
    el = time.perf_counter() - t0
    auc = float(roc_auc_score(yte, mb.predict(h, xte, feature_major=True)))
    out["higgs_like_10m_goss"] = {
        "workload": "HIGGS-like 10M x 28 (synthetic), logistic, GOSS top 0.2 / other 0.1",
        "trees": trees, "fit_seconds": el, "auc": auc,
        "note": "whole macboost_train call; the reference's GOSS run (1.9 s, real HIGGS) "
                "is not comparable"}
    log(f"HIGGS-like 10M GOSS: {trees} trees in {el:.3f}s, AUC {auc:.4f}")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--rows", type=int, default=10_000_000)
    ap.add_argument("--cols", type=int, default=100)
    ap.add_argument("--cpu-rows", type=int, default=2_000_000)
    ap.add_argument("--cpu-trees", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the leaf-wise, predict and TreeSHAP measurements")
    ap.add_argument("--extra-trees", type=int, default=100)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported "
              "(the library has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)

    import macboost_amd as mb

    rows, cols = args.rows, args.cols
    log(f"generating Friedman #1 {rows} x {cols}")
    t0 = time.perf_counter()
    x, y = mb.friedman(rows, cols, 42)
    log(f"data in {time.perf_counter() - t0:.2f}s")
    params = {"num_trees": args.steps + args.warmup, "max_depth": 6, "num_bins": 256,
              "learning_rate": 0.1}
    t0 = time.perf_counter()
    tr = mb.Trainer(params, x, y, feature_major=True)
    t_setup = time.perf_counter() - t0
    t_edges, t_bin = tr.setup_seconds()
    log(f"setup {t_setup:.2f}s (edges {t_edges:.2f}s, upload+bin {t_bin:.2f}s)")
    tr.grow(args.warmup)
    log(f"warm-up {args.warmup} trees done")
    tr.profile(True)
    t0 = time.perf_counter()
    tr.grow(args.steps)
    elapsed = time.perf_counter() - t0
    launches, hist_ms, hist_bytes = tr.hist_stats()
    built, active, level_ms = tr.level_stats(6)
    value = args.steps / elapsed
    log(f"{args.steps} trees in {elapsed:.3f}s = {value:.1f} trees/s; hist {launches} launches "
        f"{hist_ms:.1f} ms")
    h = tr.booster()
    # quality check: held-out RMSE (README.md:73 reports 1.033 for the reference)
    xv, yv = mb.friedman(200_000, cols, 42 + 999)
    pv = mb.predict(h, xv, feature_major=True)
    rmse = float(np.sqrt(np.mean((pv.astype(np.float64) - yv) ** 2)))
    log(f"valid RMSE {rmse:.4f} after {args.steps + args.warmup} trees")
    tr.close()
    extras = None if args.no_extras else measure_extras(mb, x, y, cols, args.extra_trees,
                                                        not args.no_cpu)

    achieved = hist_bytes / (hist_ms / 1e3) / 1e9 if hist_ms > 0 else None
    per_launch_bytes = hist_bytes / launches if launches else None
    traffic = None
    tfile = ROOT / "profiles" / "k_hist_traffic_friedman10m.json"
    if tfile.exists() and launches:
        # HBM bytes per k_hist launch from the committed rocprofv3 --pmc summary:
        # measured read bytes per built row x this run's built rows per launch,
        # plus the measured partial write-back per launch
        tj = json.loads(tfile.read_text())
        if (tj.get("profile_rows"), tj.get("profile_cols")) == (rows, cols):
            traffic = (tj["fetch_bytes_per_built_row"] * float(sum(built[:6])) / launches
                       + tj["write_bytes_per_launch"])
    roofline = {
        "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBS if achieved else None, "traffic": traffic,
        "kernel": "k_hist", "launches": launches, "avg_launch_ms": hist_ms / launches if launches else None,
        "algorithmic_bytes_per_launch": per_launch_bytes,
        "levels": [{"level": d, "built_rows_per_tree": float(built[d]) / args.steps,
                    "ms_per_tree": float(level_ms[d]) / args.steps,
                    "GB/s": (float(built[d]) * (cols + 4) / (level_ms[d] / 1e3) / 1e9
                             if level_ms[d] > 0 else None)} for d in range(6)],
    }
    for lv in roofline["levels"]:
        log(f"level {lv['level']}: {lv['built_rows_per_tree']:.0f} rows/tree, "
            f"{lv['ms_per_tree'] * 1e3:.1f} us/tree, {lv['GB/s'] or 0:.0f} GB/s")
    cpu = None
    if not args.no_cpu:
        cr = min(args.cpu_rows, rows)
        log(f"cpu baseline: oracle on {cr} rows, {args.cpu_trees} tree(s)")
        t_cbin, t_cfit = cpu_baseline(x, y, cr, cols, args.cpu_trees)
        per_tree_full = t_cfit / args.cpu_trees * (rows / cr)
        cpu = {"value": 1.0 / per_tree_full, "unit": "trees/s", "cores": 1, "kind": "port",
               "sample": f"{args.cpu_trees} depth-6 tree(s) on the first {cr} of {rows} rows "
                         f"x {cols} features (binned once, {t_cbin:.1f}s, untimed), "
                         f"{t_cfit:.2f}s, scaled linearly to {rows} rows"}
        log(f"cpu {t_cfit:.2f}s for {args.cpu_trees} tree(s) on {cr} rows")
    fit_total = t_setup + elapsed / args.steps * 100
    out = {
        "metric": "trees/s fitting 10M×100 depth-6; histogram HBM GB/s as % of peak",
        "value": value, "unit": "trees/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": value / REFERENCE_TREES_PER_S,
        "dtype": "u8 bins, int64 histograms, f32 gains", "data": "synthetic",
        "config": {"workload": "friedman1-regression-levelwise", "rows": rows, "features": cols,
                   "bins": 256, "max_depth": 6, "learning_rate": 0.1, "objective": "l2",
                   "parallelism": "single-gpu"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "rows_per_s": rows * value,
        "fit_seconds_100_trees_incl_binning": fit_total,
        "vs_baseline_basis": "value / 25.6 trees/s (100 trees in 3.9 s on an M4 Max, README.md:73). "
                             "The reference's 3.9 s also includes binning; on that basis the ratio "
                             f"is 3.9 s / fit_seconds_100_trees_incl_binning = {3.9 / fit_total:.1f}",
        "setup_seconds": {"edges_device": t_edges, "upload_and_bin": t_bin, "total": t_setup},
        "valid_rmse": rmse,
        "leafwise_predict_treeshap": extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
