#!/usr/bin/env python3
"""Benchmark of the MI355X tree-build path.

Headline (the metric's workload): Friedman #1 regression, 10M rows x 100 fp32
features, 256 bins, level-wise depth 6, lr 0.1, L2, 100 trees.  A step is one
complete macboost_train call from host memory, i.e. everything
FitTimings.total covers (Booster.swift:505-506, :564-565, :1699): the 4 GB
host-to-device copy of X, device quantile edges, binning, the 100 trees and
the readback of the model.  W untimed steps, then K timed steps, each timed
on its own; value = 100 / the median step (trees/s).  The held-out RMSE after
those 100 trees is reported (the reference: 1.033, README.md:73).

Also reported:
* roofline: the histogram kernel, algorithmic bytes (sum over built nodes of
  rows * (features + 4)) over its HIP-event time on the trainer's stream,
  measured inside the timed steps; traffic from the committed rocprofv3
  FETCH_SIZE / WRITE_SIZE summary;
* the same fit with X already resident in HBM (mbk_fit), and the rate with
  the binned matrix resident (trees only);
* the small (20k x 100, 64 bins) and 1M x 100 Friedman workloads, the NaN +
  categorical workload with per-iteration validation, the HIGGS-like
  logistic workload plain and with GOSS, and leaf-wise growth (63 leaves)
  with 500k-row batch predict and 200k-row TreeSHAP;
* CPU baselines on this host: the oracle (tests/oracle_lib.py, OpenMP over
  the host cores, results identical at any thread count) on the headline
  workload (binning + a prefix of trees, extrapolated), the 20k and 1M
  workloads on one core in full, and batch predict and TreeSHAP on every
  core.

Prints one JSON line on stdout; progress goes to stderr.
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
REFERENCE_TREES_PER_S = 100 / 3.9    # 100 trees in 3.9 s on an M4 Max (README.md:73)
LEVELWISE = {"max_depth": 6, "num_bins": 256, "learning_rate": 0.1}
PROFILE_EVERY = 5    # default: histogram launches of every 5th timed tree carry timestamps


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def rmse(p, y):
    d = np.asarray(p, np.float64) - np.asarray(y, np.float64)
    return float(np.sqrt(np.mean(d * d)))


def time_fits(ctx, params, x_dev, rows, cols, y, n, row_major=False, eval_set=None):
    """n fits through mbk_fit; (seconds per fit, the last booster)."""
    h = None
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(n):
        h = ctx.fit(params, x_dev, rows, cols, y, row_major=row_major, eval_set=eval_set)
    return (time.perf_counter() - t0) / n, h


def headline(mb, ctx, args):
    rows, cols, trees = args.rows, args.cols, 100
    log(f"generating Friedman #1 {rows} x {cols} (seed 42)")
    x, y = mb.friedman(rows, cols, 42)
    params = dict(LEVELWISE, num_trees=trees)
    for _ in range(args.warmup):
        mb.train(params, x, y, feature_major=True)
    log(f"{args.warmup} warm-up steps done")
    # the histogram launches of every PROFILE_EVERY-th tree carry their own
    # dispatch timestamps (a timestamped launch costs a few microseconds more)
    mb.profile_train(True, every=args.profile_every)
    times, h = [], None
    ctx.sync()
    t_all = time.perf_counter()
    for k in range(args.steps):
        t0 = time.perf_counter()
        h = mb.train(params, x, y, feature_major=True)     # returns after the model readback
        times.append(time.perf_counter() - t0)
        log(f"step {k}: {times[-1] * 1e3:.1f} ms")
    ctx.sync()
    total = time.perf_counter() - t_all
    mb.profile_train(False)
    stats = mb.train_hist_stats(16)
    med = float(np.median(times))
    value = trees / med
    log(f"{args.steps} complete fits of {trees} trees from host memory: median "
        f"{med * 1e3:.1f} ms (mean {total / args.steps * 1e3:.1f}) = {value:.1f} trees/s")
    xv, yv = mb.friedman(200_000, cols, 42 + 999)
    valid = rmse(mb.predict(h, xv, feature_major=True), yv)
    log(f"held-out RMSE after {mb.num_trees(h)} trees: {valid:.4f}")
    return x, y, times, total, value, valid, stats


def x_resident(mb, ctx, x, y, rows, cols, steps):
    """The same fit through mbk_fit with X already in HBM (no PCIe copy)."""
    x_dev = ctx.upload(x)
    ctx.sync()
    params = dict(LEVELWISE, num_trees=100)
    ctx.fit(params, x_dev, rows, cols, y)
    sec, _ = time_fits(ctx, params, x_dev, rows, cols, y, steps)
    log(f"X resident in HBM: {sec * 1e3:.1f} ms per fit = {100 / sec:.1f} trees/s")
    return x_dev, {"fit_seconds": sec, "trees_per_s": 100 / sec, "fits": steps,
                   "note": "mbk_fit on device-resident features: edges, binning, trees, "
                           "model readback; no host-to-device copy of X"}


def roofline_of(stats, rows, cols, steps, trees, every):
    launches, hist_ms, hist_bytes, built, level_ms = stats
    achieved = hist_bytes / (hist_ms / 1e3) / 1e9 if hist_ms > 0 else None
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
    n_trees = steps * ((trees + every - 1) // every)   # the timed trees
    levels = []
    for d in range(6):
        gbs = float(built[d]) * (cols + 4) / (level_ms[d] / 1e3) / 1e9 if level_ms[d] > 0 else None
        levels.append({"level": d, "built_rows_per_tree": float(built[d]) / n_trees,
                       "us_per_tree": float(level_ms[d]) / n_trees * 1e3, "GB/s": gbs})
        log(f"level {d}: {built[d] / n_trees:.0f} rows/tree, "
            f"{level_ms[d] / n_trees * 1e3:.1f} us/tree, {gbs or 0:.0f} GB/s")
    return {
        "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBS if achieved else None, "traffic": traffic,
        "kernel": "k_hist", "launches": launches,
        "timed_launches": f"every histogram launch of every {every}th tree of the timed fits",
        "avg_launch_ms": hist_ms / launches if launches else None,
        "algorithmic_bytes_per_launch": hist_bytes / launches if launches else None,
        "algorithmic_bytes_definition": "sum over built nodes of rows * (features + 4)",
        "traffic_over_algorithmic": (traffic / (hist_bytes / launches)
                                     if traffic and launches else None),
        "levels": levels,
    }


def headline_extras(mb, x, y, rows, cols):
    out = {}
    params = dict(LEVELWISE, num_trees=100)
    tr = mb.Trainer(dict(params, num_trees=110), x, y, feature_major=True)
    e, b = tr.setup_seconds()
    out["setup_seconds"] = {"upload": b, "edges_and_binning": e}
    tr.grow(10)
    t0 = time.perf_counter()
    tr.grow(100)
    el = time.perf_counter() - t0
    tr.close()
    out["trees_per_s_bins_resident"] = 100 / el
    log(f"trees only, bins resident: {100 / el:.1f} trees/s (setup: upload {b * 1e3:.1f} ms, "
        f"edges + binning {e * 1e3:.1f} ms)")
    return out


def small_and_1m(mb, ctx, with_cpu, c2_cpu_full=False):
    """The 20k x 100 (64 bins) and 1M x 100 Friedman workloads, 100 trees.  The
    oracle runs on one core: the 20k workload in full, the 1M one with a
    20-tree prefix extrapolated (in full with c2_cpu_full)."""
    out = {}
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    for name, rows, nb, test_rows, ref in (
            ("friedman_20k", 20_000, 64, 20_000, {"reference_trees_per_s": 947.0,
                                                  "reference_source": "README.md:74 (256 bins)"}),
            ("friedman_1m", 1_000_000, 256, 200_000, {"reference_fit_seconds": 0.49,
                                                      "reference_valid_rmse": 1.038,
                                                      "reference_source": "README.md:71"})):
        x, y = mb.friedman(rows, 100, 42)
        xt, yt = mb.friedman(test_rows, 100, 42 + 999)
        params = {"num_trees": 100, "max_depth": 6, "num_bins": nb, "learning_rate": 0.1}
        d = ctx.upload(x)
        ctx.fit(params, d, rows, 100, y)
        sec, h = time_fits(ctx, params, d, rows, 100, y, 5)
        t0 = time.perf_counter()
        mb.train(params, x, y, feature_major=True)
        pcie = time.perf_counter() - t0
        r = {"workload": f"Friedman #1 {rows} x 100, {nb} bins, 100 trees, level-wise depth 6",
             "fit_seconds": sec, "trees_per_s": 100 / sec, "rows_per_s": rows * 100 / sec,
             "fit_seconds_pcie_inclusive": pcie,
             "valid_rmse": rmse(mb.predict(h, xt, feature_major=True), yt), **ref}
        log(f"{name}: {sec * 1e3:.1f} ms per 100-tree fit ({100 / sec:.0f} trees/s), "
            f"PCIe-inclusive {pcie * 1e3:.1f} ms, valid RMSE {r['valid_rmse']:.4f}")
        if with_cpu:
            # one thread: the small workload in full; the 1M one binning and a
            # 20-tree prefix, extrapolated to 100 trees (or in full)
            small = rows <= 20_000
            O.set_threads(1)
            threads, ntrees = O.get_threads(), 100 if small or c2_cpu_full else 20
            t0 = time.perf_counter()
            edges = O.compute_edges(x, nb)
            bins = O.bin_matrix(x, edges, nb)
            t_bin = time.perf_counter() - t0
            t0 = time.perf_counter()
            m = O.fit(bins, y, edges=edges, num_bins=nb, num_trees=ntrees, max_depth=6)
            t_fit = time.perf_counter() - t0
            O.set_threads(0)
            fit100 = t_bin + t_fit * 100 / ntrees
            r["cpu_oracle"] = {"fit_seconds": fit100, "trees_per_s": 100 / fit100,
                               "threads": threads, "binning_seconds": t_bin,
                               "trees_timed": ntrees, "trees_seconds": t_fit,
                               "note": "edges + binning + 100 trees in full" if ntrees == 100 else
                                       "edges + binning + 20 trees timed, 100 extrapolated"}
            if ntrees == 100:
                r["cpu_oracle"]["valid_rmse"] = rmse(
                    O.predict(m.forest, m.base_score, nb, xt), yt)
            log(f"{name}: oracle on {threads} thread(s): 100-tree fit {fit100:.2f}s")
        out[name] = r
    return out


def leafwise_predict_shap(mb, ctx, x_dev, rows, cols, y, with_cpu):
    """63-leaf best-first growth on the headline data, then batch predict of
    500k held-out rows and TreeSHAP of 200k rows with that model."""
    sys.path.insert(0, str(ROOT / "tests"))
    import model_io
    import oracle_lib as O
    out = {}
    params = {"num_trees": 100, "max_depth": 6, "num_bins": 256, "num_leaves": 63}
    ctx.fit(dict(params, num_trees=5), x_dev, rows, cols, y)
    sec, h = time_fits(ctx, params, x_dev, rows, cols, y, 2)
    out["leafwise_fit"] = {"workload": "Friedman #1 10M x 100, 63 leaves, depth 6, 256 bins, "
                                       "100 trees, X resident in HBM",
                           "fit_seconds": sec, "trees_per_s": 100 / sec}
    log(f"leaf-wise 63 leaves: {sec * 1e3:.1f} ms per 100-tree fit = {100 / sec:.1f} trees/s")
    obj = model_io.saved_model(h)
    forest = model_io.forest_from_json(obj)
    base, nb = obj["baseScore"], obj["numBins"]
    xp, _ = mb.friedman(500_000, cols, 42 + 999)
    mb.predict(h, xp[:, :1000], feature_major=True)
    t0 = time.perf_counter()
    pp = mb.predict(h, xp, feature_major=True)
    el = time.perf_counter() - t0
    pred = {"rows": 500_000, "trees": int(forest.num_trees), "seconds": el,
            "rows_per_s": 500_000 / el,
            "note": "through macboost_predict: X copied host -> HBM and the output back"}
    if with_cpu:
        t1 = time.perf_counter()
        want = O.predict(forest, base, nb, xp)
        cpu_el = time.perf_counter() - t1
        pred["bit_exact_vs_oracle_all_rows"] = bool(np.array_equal(pp, want))
        pred["cpu_oracle"] = {"seconds": cpu_el, "rows_per_s": 500_000 / cpu_el,
                              "threads": O.get_threads(),
                              "note": "predictCPU restated, 16,384-row chunks over the threads"}
    out["predict"] = pred
    log(f"predict 500k x {forest.num_trees} trees: {el * 1e3:.1f} ms")
    xs = np.ascontiguousarray(xp[:, :200_000])
    mb.predict_contrib(h, xs[:, :1000], feature_major=True)
    t0 = time.perf_counter()
    c = mb.predict_contrib(h, xs, feature_major=True)
    el = time.perf_counter() - t0
    shap = {"rows": 200_000, "trees": int(forest.num_trees), "seconds": el,
            "row_trees_per_s": 200_000 * forest.num_trees / el,
            "reference_row_trees_per_s": 50e6, "reference_source": "README.md:35-36"}
    if with_cpu:
        pick = np.arange(0, 200_000, 100)
        t1 = time.perf_counter()
        ref = O.treeshap(forest, base, nb, np.ascontiguousarray(xs[:, pick]))
        cpu_el = time.perf_counter() - t1
        shap["within_1e-5_rel_vs_oracle_2000_rows"] = bool(
            np.allclose(c[pick], ref, rtol=1e-5, atol=1e-6))
        shap["cpu_oracle"] = {"rows": len(pick), "seconds": cpu_el,
                              "row_trees_per_s": len(pick) * forest.num_trees / cpu_el,
                              "threads": O.get_threads(),
                              "note": "recursive fp64 TreeSHAP, 512-row chunks over the threads"}
    out["treeshap"] = shap
    log(f"TreeSHAP 200k x {forest.num_trees} trees: {el * 1e3:.1f} ms")
    return out


def mixed_1m(mb, ctx):
    """Whole fits (X resident) on the NaN + categorical workload."""
    sys.path.insert(0, str(ROOT / "tests"))
    import datasets as D
    out = {}
    x, y, cats = D.c3_mixed(1_000_000, 42)
    xv, yv, _ = D.c3_mixed(200_000, 42 + 999)
    params = {"num_trees": 100, "max_depth": 6, "num_bins": 256, "categorical_features": cats}
    d = ctx.upload(x)
    ctx.fit(dict(params, num_trees=2), d, 1_000_000, 100, y)
    sec, h = time_fits(ctx, params, d, 1_000_000, 100, y, 2, eval_set=(xv.T, yv))
    out["nan_categorical_1m"] = {
        "workload": "Friedman #1 1M x 100, 20 categorical columns (cardinality 2..64), 20% NaN, "
                    "200k validation rows scored after every tree, 100 trees",
        "fit_seconds": sec, "valid_rmse": float(mb.eval_history(h)[-1]),
        "reference_fit_seconds": 0.76, "reference_source": "README.md:72 (other generator)"}
    log(f"NaN+categorical 1M: {sec * 1e3:.1f} ms per fit, valid RMSE "
        f"{out['nan_categorical_1m']['valid_rmse']:.4f}")
    return out


def higgs(mb, ctx):
    """Whole fits (X resident) on the HIGGS-like workload, plain and with GOSS."""
    sys.path.insert(0, str(ROOT / "tests"))
    import datasets as D
    from sklearn.metrics import roc_auc_score
    out = {}
    x, y = D.c4_higgs_like(10_500_000, 42)
    n = 10_000_000
    xtr, ytr = np.ascontiguousarray(x[:, :n]), y[:n]
    xte, yte = np.ascontiguousarray(x[:, n:]), y[n:]
    del x
    d = ctx.upload(xtr)
    params = {"num_trees": 100, "max_depth": 6, "num_bins": 256, "objective": "binary"}
    for key, extra, ref in (("higgs_like_10m", {}, 2.8),
                            ("higgs_like_10m_goss", {"goss": True}, 1.9)):
        p = dict(params, **extra)
        ctx.fit(dict(p, num_trees=12), d, n, 28, ytr)
        sec, h = time_fits(ctx, p, d, n, 28, ytr, 2)
        auc = float(roc_auc_score(yte, mb.predict(h, xte, feature_major=True)))
        out[key] = {"workload": "HIGGS-like 10M x 28 (synthetic), logistic, 100 trees"
                                + (", GOSS top 0.2 / other 0.1" if extra else ""),
                    "fit_seconds": sec, "auc": auc, "reference_fit_seconds": ref,
                    "reference_source": "README.md:62-63 (real HIGGS: not comparable)"}
        log(f"{key}: {sec * 1e3:.1f} ms per fit, AUC {auc:.4f}")
    out["goss_speedup"] = out["higgs_like_10m"]["fit_seconds"] / \
        out["higgs_like_10m_goss"]["fit_seconds"]
    return out


def cpu_baseline(x, y, rows, cols, prefix):
    """The oracle on the headline workload: edges + binning of every row and
    `prefix` trees, on every host thread; 100-tree fit time extrapolated."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    O.set_threads(0)
    threads = O.get_threads()
    t0 = time.perf_counter()
    edges = O.compute_edges(x, 256)
    bins = O.bin_matrix(x, edges, 256)
    t_bin = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.fit(bins, y, edges=edges, num_trees=prefix, max_depth=6, num_bins=256)
    t_fit = time.perf_counter() - t0
    fit100 = t_bin + t_fit / prefix * 100
    log(f"cpu oracle ({threads} threads): binning {t_bin:.2f}s, {prefix} trees {t_fit:.2f}s")
    return {"value": 100 / fit100, "unit": "trees/s", "cores": threads, "kind": "port",
            "sample": f"oracle (C + OpenMP, {threads} threads, host nproc {os.cpu_count()}) on "
                      f"all {rows} x {cols} rows: edges + binning {t_bin:.2f}s and {prefix} "
                      f"depth-6 trees {t_fit:.2f}s, timed; 100-tree fit time extrapolated as "
                      f"binning + 100 x per-tree = {fit100:.1f}s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10, help="timed 100-tree fits")
    ap.add_argument("--warmup", type=int, default=2, help="untimed 100-tree fits")
    ap.add_argument("--rows", type=int, default=10_000_000)
    ap.add_argument("--cols", type=int, default=100)
    ap.add_argument("--cpu-trees", type=int, default=10)
    ap.add_argument("--profile-every", type=int, default=PROFILE_EVERY,
                    help="time the histogram launches of every k-th tree of the timed fits")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--c2-cpu-full", action="store_true",
                    help="time the 1M-row workload's oracle on one core for all 100 trees "
                         "(about 2 minutes)")
    ap.add_argument("--no-extras", action="store_true",
                    help="only the headline fits (no other workloads)")
    ap.add_argument("--only", choices=["small_1m", "mixed", "higgs"],
                    help="run one other workload alone and print its record instead of the "
                         "headline line (for profiling that workload)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported "
              "(the library has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)

    import macboost_amd as mb
    ctx = mb.Context(0)
    if args.only:
        run = {"small_1m": lambda: small_and_1m(mb, ctx, not args.no_cpu, args.c2_cpu_full),
               "mixed": lambda: mixed_1m(mb, ctx), "higgs": lambda: higgs(mb, ctx)}[args.only]
        print(json.dumps({"only": args.only, **run()}), flush=True)
        return
    rows, cols = args.rows, args.cols
    x, y, times, total, value, valid, stats = headline(mb, ctx, args)
    roofline = roofline_of(stats, rows, cols, args.steps, 100, args.profile_every)
    med = float(np.median(times))
    x_dev, resident = x_resident(mb, ctx, x, y, rows, cols, 5)
    extras = {"x_resident": resident}
    if not args.no_extras:
        extras.update(headline_extras(mb, x, y, rows, cols))
        extras["leafwise_predict_treeshap"] = leafwise_predict_shap(
            mb, ctx, x_dev, rows, cols, y, not args.no_cpu)
        extras["small_and_1m"] = small_and_1m(mb, ctx, not args.no_cpu, args.c2_cpu_full)
        extras["mixed_and_higgs"] = {**mixed_1m(mb, ctx), **higgs(mb, ctx)}
    cpu = None if args.no_cpu else cpu_baseline(x, y, rows, cols, args.cpu_trees)
    out = {
        "metric": "trees/s fitting 10M×100 depth-6; histogram HBM GB/s as % of peak",
        "value": value, "unit": "trees/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": med * 1e3,
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": value / REFERENCE_TREES_PER_S,
        "dtype": "u8 bins, int64 histograms, f32 gains", "data": "synthetic",
        "config": {"workload": "friedman1-regression-levelwise", "rows": rows, "features": cols,
                   "bins": 256, "max_depth": 6, "learning_rate": 0.1, "objective": "l2",
                   "trees_per_fit": 100, "parallelism": "single-gpu",
                   "step": "one complete 100-tree macboost_train from host memory: the 4 GB "
                           "host-to-device copy of X, device edges, binning, trees, model "
                           "readback"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "rows_per_s": rows * value,
        "step_ms": [t * 1e3 for t in times],
        "mean_ms_per_step": total / args.steps * 1e3,
        "fit_seconds_100_trees": med,
        "valid_rmse_after_100_trees": valid,
        "reference_valid_rmse": 1.033,
        "vs_baseline_basis": "value / (100 trees / 3.9 s), the reference's 10M x 100 fit on an "
                             "M4 Max (README.md:73), which also copies X into a device buffer "
                             "and bins it",
        "host_nproc": os.cpu_count(),
        **extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
