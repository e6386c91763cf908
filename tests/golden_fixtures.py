"""Inputs of the reference's golden-bit fixtures, restated from
`tests/test_golden_bits.mojo:7928-8115` (ajhendel/mojoboost) and
`tests/support.mojo:22-42`: every feature value is
`uniform(k + seed)` over the column-major index `k = f * n_rows + r`.

Only the generators live here; the expected outputs are the data fixture
tests/golden/golden_bits.json.
"""
import json
from fractions import Fraction
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden_bits.json"
M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(counter: np.ndarray) -> np.ndarray:
    return (splitmix64(counter) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def features(n_rows: int, n_features: int, seed: int) -> np.ndarray:
    k = np.arange(n_rows * n_features, dtype=np.uint64) + np.uint64(seed)
    return uniform(k)


def fma(a: float, b: float, c: float) -> float:
    """Correctly rounded a*b+c (exact rational arithmetic, one rounding)."""
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def regression_target(x: np.ndarray, n_rows: int) -> np.ndarray:
    """`3*x0 - 2*x1 + x2*x3 + 0.5*(x2 - 0.5)^2` as the reference evaluated
    it: Mojo's default `--fp-mode contract=fast` fuses each `a*b + c` into an
    FMA (reference docs/NUMERICS.md section 3.3), and the first subtraction
    fuses the left product: fma(3, x0, -(2*x1)). This contraction pattern is
    the one that reproduces every golden raw score bit."""
    x0, x1, x2, x3 = (x[i * n_rows:(i + 1) * n_rows] for i in range(4))
    y = np.empty(n_rows)
    for r in range(n_rows):
        a, b, c, d = float(x0[r]), float(x1[r]), float(x2[r]), float(x3[r])
        s = fma(3.0, a, -(2.0 * b))
        s = fma(c, d, s)
        q = 0.5 * (c - 0.5)
        y[r] = fma(q, c - 0.5, s)
    return y


def load_golden():
    return json.loads(GOLDEN.read_text())


def fixture(name: str):
    """Returns (x_cm, n_rows, n_features, labels, binning, params_kw)."""
    if name == "l2":
        n, f = 200, 8
        x = features(n, f, 0)
        return x, n, f, regression_target(x, n), ("equal", 32), dict(
            objective=0, num_iterations=8, learning_rate=0.3, num_leaves=8,
            min_data_in_leaf=5, lambda_l2=1.0, min_sum_hessian=1e-3)
    if name == "logit":
        n, f = 200, 8
        x = features(n, f, 10_000)
        y = np.empty(n)
        for r in range(n):
            s = fma(2.0, float(x[r]), -float(x[n + r]))
            s = fma(float(x[2 * n + r]), float(x[3 * n + r]), s)
            y[r] = 1.0 if s > 1.0 else 0.0
        return x, n, f, y, ("equal", 32), dict(
            objective=1, num_iterations=8, learning_rate=0.3, num_leaves=8,
            min_data_in_leaf=5, lambda_l2=1.0, min_sum_hessian=1e-3)
    if name == "multi":
        n, f, k = 150, 6, 3
        x = features(n, f, 20_000)
        y = np.empty(n)
        for r in range(n):
            s = fma(0.3, float(x[n + r]), 0.5 * float(x[r]))
            s = fma(0.2, float(x[2 * n + r]), s)
            c = int(s * float(k))
            y[r] = k - 1 if c >= k else c
        return x, n, f, y, ("equal", 32), dict(
            objective=2, num_class=3, num_iterations=4, learning_rate=0.3, num_leaves=6,
            min_data_in_leaf=5, lambda_l2=1.0, min_sum_hessian=1e-3)
    if name == "bagged":
        n, f = 200, 8
        x = features(n, f, 0)
        return x, n, f, regression_target(x, n), ("equal", 32), dict(
            objective=0, num_iterations=8, learning_rate=0.3, num_leaves=8,
            min_data_in_leaf=5, lambda_l2=1.0, min_sum_hessian=1e-3,
            bagging_fraction=0.6, bagging_freq=1, bagging_seed=7)
    if name == "ffrac":
        n, f = 200, 12
        x = features(n, f, 30_000)
        return x, n, f, regression_target(x, n), ("equal", 32), dict(
            objective=0, num_iterations=8, learning_rate=0.3, num_leaves=8,
            min_data_in_leaf=5, lambda_l2=1.0, min_sum_hessian=1e-3, feature_fraction=0.5)
    if name == "large":
        n, f = 12_000, 6
        x = features(n, f, 90_000)
        r = np.arange(n)
        x[4 * n:5 * n] = (r % 16).astype(np.float64)
        col5 = np.where(r % 97 == 0, 8 + (r // 97) % 32, r % 8).astype(np.float64)
        x[5 * n:6 * n] = col5
        return x, n, f, regression_target(x, n), ("fit", 255), dict(
            objective=0, num_iterations=8, learning_rate=0.3, num_leaves=31,
            min_data_in_leaf=20, lambda_l2=1.0, min_sum_hessian=1e-3)
    if name == "misscat":
        # _fixture_misscat (tests/test_golden_bits.mojo:8072-8113): feature 1
        # missing on every seventh row, feature 2 an integer code in [0, 6)
        # fitted as a categorical, the target additive in both. 2 * x0 is
        # exact, so no contraction choice moves the target's bits.
        n, f = 200, 5
        x = features(n, f, 40_000)
        r = np.arange(n)
        x[1 * n:2 * n][r % 7 == 0] = np.nan
        x[2 * n:3 * n] = np.floor(x[2 * n:3 * n] * 6.0)
        weight = np.array([0.0, 1.5, -1.0, 0.7, -2.0, 2.5])
        y = np.empty(n)
        for i in range(n):
            x1 = float(x[n + i])
            v = 2.0 * float(x[i])
            v += 0.5 if np.isnan(x1) else x1
            v += float(weight[int(x[2 * n + i])])
            y[i] = v
        return x, n, f, y, ("fit_cat", 32, [2]), dict(
            objective=0, num_iterations=8, learning_rate=0.3, num_leaves=8,
            min_data_in_leaf=5, lambda_l2=1.0, min_sum_hessian=1e-3, lambda_l1=0.0,
            max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=2.0, cat_l2=10.0,
            min_data_per_group=5)
    raise KeyError(name)


def bits_hex(a: np.ndarray) -> list:
    return ["%016x" % v for v in np.asarray(a, np.float64).view(np.uint64)]


def record(model, bins_cm, n_rows, n_features):
    """The reference's _record: tree ints, node value bits, raw, pred bits."""
    ints = [model.n_trees]
    vals = []
    for t in range(model.n_trees):
        tr = model.tree(t)
        ints.append(len(tr["feature"]))
        for i in range(len(tr["feature"])):
            ints += [int(tr["feature"][i]), int(tr["threshold"][i]), int(tr["left"][i]),
                     int(tr["right"][i])]
        vals += bits_hex(tr["value"])
    raw, pred = model.predict_binned(bins_cm, n_rows, n_features)
    return ints, vals, bits_hex(raw), bits_hex(pred)
