"""Sample weights in the oracle (boosting._fill_grad_hess_into,
src/mojotrees/boosting.mojo:676-811; boosting._base_score, :521-568;
train_multiclass's class priors, :4167-4250), pinned by what the weighting
fixes independently of the formula:

- unit weights reproduce the unweighted derivatives bit for bit;
- the hessian floor (1e-16) comes before the weight, so a tiny weight on a
  saturated row scales the floor instead of being floored itself;
- on the fp32 path, zero-weight rows add exact zeros to every histogram sum,
  so a fit with some rows at weight 0 grows the same trees, leaf values and
  base score, bit for bit, as a fit on the other rows alone (min_data_in_leaf
  1, so row counts decide nothing); a weight dropped from the gradient, the
  hessian or the base score breaks this;
- integer weights act as repeated rows in the base score (dyadic labels keep
  the sums exact).
"""
import numpy as np
import pytest

import oracle_lib as O


def test_unit_weights_match_unweighted_derivatives():
    rng = np.random.default_rng(0)
    n = 2000
    raw = rng.normal(size=n) * 3
    for obj, y in ((0, rng.normal(size=n)), (1, (rng.uniform(size=n) < 0.4).astype(float))):
        g0, h0 = O.grad_hess(obj, raw, y)
        g1, h1 = O.grad_hess_w(obj, raw, y, np.ones(n))
        assert np.array_equal(g0, g1) and np.array_equal(h0, h1)


def test_hessian_floor_comes_before_the_weight():
    # p(1 - p) of raw 40 is far below 1e-16: the unweighted hessian is the
    # floor, and a weight of 1e-20 scales that floor to 1e-36 (fp32 keeps it)
    raw = np.array([40.0, -40.0, 0.0])
    y = np.array([1.0, 0.0, 1.0])
    w = np.array([1e-20, 3.0, 0.5])
    g, h = O.grad_hess_w(1, raw, y, w)
    assert h[0] == np.float32(1e-20 * 1e-16) and h[0] < 1e-30
    assert h[1] == np.float32(3.0 * 1e-16)
    assert h[2] == np.float32(0.5 * 0.25) and g[2] == np.float32(0.5 * (0.5 - 1.0))


def test_zero_weights_match_fit_on_the_other_rows():
    rng = np.random.default_rng(1)
    n, f, nb = 6000, 5, 32
    x = rng.normal(size=(f, n))
    bins = np.clip(((x + 3) / 6 * nb).astype(int), 0, nb - 1).astype(np.uint8)
    z = x[0] - 0.7 * x[1] * x[2]
    keep = rng.uniform(size=n) < 0.7
    w = keep.astype(float)
    for obj in (0, 1):
        y = z + 0.1 * rng.normal(size=n) if obj == 0 else \
            (rng.uniform(size=n) < 1 / (1 + np.exp(-z))).astype(float)
        kw = dict(objective=obj, num_iterations=4, num_leaves=12, min_data_in_leaf=1, lambda_l2=1.0,
                  learning_rate=0.2, use_quantized_grad=0)
        p, _w = O.weighted_params(w, **kw)
        full = O.train(bins.ravel(), n, f, nb, y, p)
        sub_bins = np.ascontiguousarray(bins[:, keep])
        m = int(keep.sum())
        sub = O.train(sub_bins.ravel(), m, f, nb, y[keep], O.default_params(**kw))
        assert full.n_trees == sub.n_trees
        assert np.array_equal(full.base.view(np.uint64), sub.base.view(np.uint64))
        for k in ("feature", "threshold", "left", "right", "default_left"):
            assert np.array_equal(getattr(full, k), getattr(sub, k)), (obj, k)
        assert np.array_equal(full.value.view(np.uint64), sub.value.view(np.uint64))
        assert np.array_equal(full.train_raw(n)[keep].view(np.uint64), sub.train_raw(m).view(np.uint64))


def test_integer_weights_act_as_repeated_rows_in_the_base_score():
    rng = np.random.default_rng(2)
    n, nb = 500, 16
    bins = rng.integers(0, nb, size=n).astype(np.uint8)
    y = rng.integers(-16, 17, size=n) / 8.0
    reps = rng.integers(0, 4, size=n)
    kw = dict(objective=0, num_iterations=1, num_leaves=2, learning_rate=0.1)
    p, _w = O.weighted_params(reps.astype(float), **kw)
    wfit = O.train(bins, n, 1, nb, y, p)
    rb = np.repeat(bins, reps)
    dup = O.train(rb, len(rb), 1, nb, np.repeat(y, reps), O.default_params(**kw))
    assert wfit.base[0] == dup.base[0] == np.sum(np.repeat(y, reps)) / reps.sum()
    # binary log-odds and multiclass priors take the weighted shares
    yb = (y > 0).astype(float)
    pb, _ = O.weighted_params(reps.astype(float), **dict(kw, objective=1))
    b = O.train(bins, n, 1, nb, yb, pb).base[0]
    share = np.sum(reps * yb) / reps.sum()
    # the reference's own log (orc_log; within 1e-9 of libm's)
    assert b == O.lib().orc_log(share / (1 - share))
    assert b == pytest.approx(np.log(share / (1 - share)), rel=1e-9)
    yc = rng.integers(0, 3, size=n).astype(float)
    pm, _ = O.weighted_params(reps.astype(float), **dict(kw, objective=2, num_class=3))
    bm = O.train(bins, n, 1, nb, yc, pm).base
    for k in range(3):
        assert bm[k] == O.lib().orc_log(np.sum(reps * (yc == k)) / reps.sum())


def test_ranker_unit_weights_and_query_bags():
    """train_ranker (ranking.mojo:690-771): unit weights change nothing; a
    query bag holds whole queries, so a fit whose bag draws every query
    (fraction just under 1) equals the unbagged fit tree for tree."""
    rng = np.random.default_rng(3)
    counts = rng.integers(1, 40, size=60).astype(np.int32)
    n = int(counts.sum())
    bins = rng.integers(0, 16, size=(3, n)).astype(np.uint8)
    y = rng.integers(0, 4, size=n).astype(float)
    kw = dict(num_iterations=4, num_leaves=7, min_data_in_leaf=3, use_quantized_grad=0)
    p0, s0 = O.rank_params(counts, **kw)
    plain = O.train(bins.ravel(), n, 3, 16, y, p0)
    p1, s1 = O.rank_params(counts, **kw)
    w = np.ones(n)
    p1.weights = w.ctypes.data
    unit = O.train(bins.ravel(), n, 3, 16, y, p1)
    assert np.array_equal(plain.value.view(np.uint64), unit.value.view(np.uint64))
    # every draw falls below 1 - 2^-40 (240 draws; any above it has odds ~2e-10)
    p2, s2 = O.rank_params(counts, bagging_fraction=1.0 - 2.0 ** -40, bagging_freq=1, **kw)
    bagged = O.train(bins.ravel(), n, 3, 16, y, p2)
    assert np.array_equal(plain.feature, bagged.feature)
    assert np.array_equal(plain.value.view(np.uint64), bagged.value.view(np.uint64))
