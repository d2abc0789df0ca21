"""Synthetic workloads for the benchmark configurations, generated from seeds
(nothing is downloaded).

- c3_mixed: Friedman #1, 100 columns. The last 20 columns (80..99) are replaced by
  integer categoricals of cardinality U{2..64}. Each category adds a seeded N(0,1)
  offset to y. Then 20% of the 80 numeric columns' entries are set to NaN, MCAR,
  after y is computed.
- c4_higgs_like: 28 HIGGS-shaped features.
  - 21 low-level columns mix N(0,1) and Exp(1), with sparse heavy tails.
  - 7 high-level columns are products and sqrt-of-sum-of-squares of low-level ones.
  - Binary labels are drawn from sigmoid(f + b), where f is a seeded depth-4
    interaction tree plus a small linear term. The intercept b is set for ~53%
    positives.

Arrays are feature-major: x has shape (cols, rows).
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def splitmix(seed: int, n: int) -> np.ndarray:
    """The first n SplitMix64 outputs of the stream seeded with `seed`
    (DataGen.swift:6-26): output k = mix(seed + k * golden), k = 1..n."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """U[0,1) as (next >> 40) * 2^-24 (DataGen.swift:16-18), float64."""
    return (splitmix(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)


def normal(seed: int, n: int) -> np.ndarray:
    """Box-Muller normals from one uniform stream, float64."""
    u = uniform(seed, 2 * n)
    u1 = np.maximum(u[0::2], 1e-12)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u[1::2])


def c3_mixed(rows: int, seed: int = 42, model_seed: int = 42):
    """Returns (x [100, rows] f32, y [rows] f32, categorical column list).
    The generating model (cardinalities and category offsets) comes from
    model_seed; the rows come from seed, so sets drawn with different seeds
    share one model."""
    import macboost_amd as mb
    x, y = mb.friedman(rows, 100, seed)
    y = y.astype(np.float64)
    cards = 2 + (splitmix(model_seed ^ 0xCA7CA7, 20) % np.uint64(63)).astype(np.int64)
    for j in range(20):
        col = 80 + j
        c = (splitmix(seed + 7919 * (j + 1), rows) % np.uint64(cards[j])).astype(np.int64)
        offsets = normal((model_seed ^ 0x0FF5E7) + 104729 * (j + 1), int(cards[j]))
        y += offsets[c]
        x[col] = c.astype(np.float32)
    miss = uniform(seed ^ 0x4E414E, 80 * rows).reshape(80, rows) < 0.2
    x[:80][miss] = np.nan
    return x, y.astype(np.float32), list(range(80, 100))


def _higgs_features(rows: int, rng) -> np.ndarray:
    x = np.empty((28, rows), np.float32)
    for f in range(21):
        v = rng.exponential(1.0, rows) if f % 3 == 2 else rng.standard_normal(rows)
        heavy = rng.random(rows) < 0.02
        v[heavy] *= 1.0 + 4.0 * rng.pareto(2.5, int(heavy.sum()))
        x[f] = v
    lo = x[:21].astype(np.float64)
    x[21] = lo[0] * lo[3]
    x[22] = lo[1] * lo[4]
    x[23] = lo[2] * lo[5]
    x[24] = np.sqrt(lo[0] ** 2 + lo[1] ** 2 + lo[2] ** 2)
    x[25] = np.sqrt(lo[3] ** 2 + lo[4] ** 2 + lo[5] ** 2)
    x[26] = np.sqrt((lo[6:10] ** 2).sum(axis=0))
    x[27] = x[24] * x[25]
    return x


def _higgs_score(xf: np.ndarray, feats, thr, leaves) -> np.ndarray:
    rows = xf.shape[1]
    node = np.zeros(rows, np.int64)
    for d in range(4):
        base = (1 << d) - 1
        f = feats[base + node]
        node = 2 * node + (xf[f, np.arange(rows)] > thr[base + node])
    return leaves[node] + 0.3 * xf[24] - 0.2 * xf[2] + 0.1 * xf[27]


def c4_higgs_like(rows: int, seed: int = 42, model_seed: int = 42):
    """Returns (x [28, rows] f32, y [rows] f32 in {0, 1}).  The label model (a
    depth-4 interaction tree, its quantile thresholds and the intercept for
    ~53% positives) comes from model_seed and a reference sample; the rows and
    label draws come from seed."""
    mrng = np.random.Generator(np.random.PCG64(model_seed))
    ref = _higgs_features(200_000, np.random.Generator(np.random.PCG64(model_seed + 1)))
    reff = ref.astype(np.float64)
    feats = mrng.integers(0, 28, size=15)
    qs = mrng.uniform(0.25, 0.75, size=15)
    thr = np.array([np.quantile(reff[feats[k]], qs[k]) for k in range(15)])
    leaves = mrng.normal(0.0, 1.5, size=16)
    s = _higgs_score(reff, feats, thr, leaves)
    lo_b, hi_b = -10.0, 10.0
    for _ in range(60):                       # intercept for ~53% positives
        b = 0.5 * (lo_b + hi_b)
        if np.mean(1.0 / (1.0 + np.exp(-(s + b)))) < 0.53:
            lo_b = b
        else:
            hi_b = b
    rng = np.random.Generator(np.random.PCG64(seed))
    x = _higgs_features(rows, rng)
    p = 1.0 / (1.0 + np.exp(-(_higgs_score(x.astype(np.float64), feats, thr, leaves) + b)))
    y = (rng.random(rows) < p).astype(np.float32)
    return x, y
