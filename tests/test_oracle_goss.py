"""Pins the oracle's GOSS (goss.mojo:294-396, the warmup of :102-157) with the
properties the reference's own GOSS tests check (tests/test_goss.mojo), on the
same inputs: counts, the multiplier, which rows are kept, ascending order,
determinism and reseeding, unbiasedness of the compensated sample, warmup and
sampled leaf counts. None of these restate the selection loop; a plausible
mistake (a flipped threshold comparison, a wrong multiplier, a stream that
ignores the round, scaling the kept rows) fails at least one."""
import numpy as np

import oracle_lib as O


def _uniform(k):
    return O.lib().orc_uniform(k)


def _features(n_rows, n_features):
    # tests/support.mojo:37-42: column-major, features[k] = uniform(k)
    return np.array([_uniform(k) for k in range(n_rows * n_features)])


def _regression_target(x, n_rows):
    # test_goss.mojo:41-50
    x0, x1, x2 = x[:n_rows], x[n_rows:2 * n_rows], x[2 * n_rows:3 * n_rows]
    return 3.0 * x0 - 2.0 * x1 + 4.0 * (x2 - 0.5) * (x2 - 0.5)


def test_selection_keeps_top_and_samples_other():
    # test_goss.mojo:61-107: 5 importance levels, 20 rows each
    grad = np.array([float(r % 5) + 1.0 for r in range(100)])
    hess = np.ones(100)
    imp = np.abs(grad * hess)
    rows, scale, g, h = O.goss_select(grad, hess, 0.2, 0.1, 3, 0)
    top = scale == 1.0
    assert top.sum() == 20 and (~top).sum() == 10 and len(rows) == 30
    assert np.all(np.abs(scale[~top] - 8.0) < 1e-12)
    assert np.all(imp[rows[top]] >= 5.0) and np.all(imp[rows[~top]] < 5.0)
    assert np.all(np.diff(rows) > 0)
    assert set(np.nonzero(imp >= 5.0)[0]) <= set(rows.tolist())
    # scaling is applied to the sampled rows only, to both g and h
    other = rows[~top]
    np.testing.assert_array_equal(g[other], grad[other] * 8.0)
    np.testing.assert_array_equal(h[other], hess[other] * 8.0)
    untouched = np.setdiff1d(np.arange(100), other)
    np.testing.assert_array_equal(g[untouched], grad[untouched])


def test_selection_is_deterministic_and_reseeds():
    # test_goss.mojo:110-140
    n = 500
    grad = np.array([2.0 * _uniform(r) - 1.0 for r in range(n)])
    hess = np.array([_uniform(1000 + r) + 0.5 for r in range(n)])
    a = O.goss_select(grad, hess, 0.2, 0.1, 7, 3)[0]
    b = O.goss_select(grad, hess, 0.2, 0.1, 7, 3)[0]
    np.testing.assert_array_equal(a, b)
    c, sc_c = O.goss_select(grad, hess, 0.2, 0.1, 7, 4)[:2]
    sc_a = O.goss_select(grad, hess, 0.2, 0.1, 7, 3)[1]
    assert (sc_a == 1.0).sum() == (sc_c == 1.0).sum()
    np.testing.assert_array_equal(a[sc_a == 1.0], c[sc_c == 1.0])  # kept half stays
    assert len(a) != len(c) or np.any(a != c)
    d = O.goss_select(grad, hess, 0.2, 0.1, 8, 3)[0]
    assert len(a) != len(d) or np.any(a != d)


def test_sample_sizes_match_the_rates():
    # other_k = floor(n * other_rate) rows are sampled whenever enough
    # small-importance rows exist (selection sampling always fills its quota)
    rng = np.random.default_rng(5)
    for n, tr, orr in [(1000, 0.2, 0.1), (777, 0.05, 0.3), (64, 0.5, 0.5), (10, 0.0, 0.3)]:
        grad = rng.standard_normal(n)
        hess = rng.uniform(0.1, 1.0, n)
        rows, scale, _, _ = O.goss_select(grad, hess, tr, orr, 1, 2)
        top_k = max(1, int(n * tr))
        other_k = min(int(n * orr), n - top_k)
        imp = np.abs(grad * hess)
        top = imp[rows] >= np.sort(imp)[::-1][top_k - 1]  # distinct importances: no ties
        assert top.sum() == top_k and (~top).sum() == other_k
        assert np.all(scale[top] == 1.0)
        if other_k:
            assert np.all(np.abs(scale[~top] - (n - top_k) / other_k) < 1e-12)


def test_compensated_sample_reproduces_full_histogram():
    # test_goss.mojo:143-194: averaged over rounds, each bin of the scaled
    # sampled gradient histogram converges to the full-data histogram
    n, nb = 400, 8
    x = _features(n, 1)
    bins = O.bin_equal_width(x, n, 1, nb)
    grad = np.array([2.0 * _uniform(7000 + r) - 1.0 for r in range(n)])
    hess = np.array([_uniform(9000 + r) + 0.25 for r in range(n)])
    full = np.bincount(bins, weights=grad, minlength=nb)
    acc = np.zeros(nb)
    for rnd in range(200):
        rows, _, g, _ = O.goss_select(grad, hess, 0.2, 0.1, 11, rnd)
        acc += np.bincount(bins[rows], weights=g[rows], minlength=nb)
    assert np.all(np.abs(acc / 200 - full) <= 0.02 * np.abs(grad).sum())


def test_zero_importance_rows_are_never_kept_on_top():
    # test_goss.mojo:197-214
    n = 200
    grad = np.array([0.0 if r % 2 == 0 else 1.0 + _uniform(r) for r in range(n)])
    hess = np.array([0.0 if r % 2 == 0 else 1.0 for r in range(n)])
    rows, scale, _, _ = O.goss_select(grad, hess, 0.2, 0.1, 3, 0)
    assert np.all(np.abs(grad[rows[scale == 1.0]] * hess[rows[scale == 1.0]]) > 0.0)


def _train(n, f, nb, lr, iters, leaves, min_data, **kw):
    x = _features(n, f)
    y = _regression_target(x, n)
    bins = O.bin_equal_width(x, n, f, nb)
    p = O.default_params(objective=O.OBJ_L2, num_iterations=iters, learning_rate=lr,
                         num_leaves=leaves, min_data_in_leaf=min_data, lambda_l2=1.0,
                         min_sum_hessian=1e-3, **kw)
    return O.train(bins, n, f, nb, y, p), bins


def test_warmup_rounds_train_on_every_row():
    # test_goss.mojo:311-333: learning_rate 0.25 -> int(1 / 0.25) = 4 warmup
    # rounds, the whole run, so the GOSS model is the full-data model
    full, _ = _train(400, 3, 32, 0.25, 4, 8, 10)
    warming, _ = _train(400, 3, 32, 0.25, 4, 8, 10, goss=1)
    np.testing.assert_array_equal(full.train_raw(400), warming.train_raw(400))
    # with 6 rounds the first 4 trees agree and the sampled rounds differ
    full6, _ = _train(400, 3, 32, 0.25, 6, 8, 10)
    goss6, _ = _train(400, 3, 32, 0.25, 6, 8, 10, goss=1)
    for t in range(4):
        np.testing.assert_array_equal(full6.tree(t)["value"], goss6.tree(t)["value"])
    assert np.any(full6.train_raw(400) != goss6.train_raw(400))


def test_training_is_deterministic_and_seeded():
    # test_goss.mojo:370-397 (warmup is int(1/lr) = 3 here, then 12 sampled rounds)
    a, _ = _train(500, 4, 32, 0.3, 15, 15, 10, goss=1, goss_seed=5)
    b, _ = _train(500, 4, 32, 0.3, 15, 15, 10, goss=1, goss_seed=5)
    np.testing.assert_array_equal(a.train_raw(500), b.train_raw(500))
    c, _ = _train(500, 4, 32, 0.3, 15, 15, 10, goss=1, goss_seed=6)
    assert np.any(a.train_raw(500) != c.train_raw(500))


def test_leaf_row_counts_come_from_the_sample():
    # test_goss.mojo:400-420: 300 rows at 0.1 + 0.1 leave 60 sampled rows,
    # so min_data_in_leaf 40 forbids every split of a sampled round, while
    # the warmup rounds (int(1 / 0.5) = 2) split freely
    m, _ = _train(300, 3, 32, 0.5, 4, 15, 40, goss=1, top_rate=0.1, other_rate=0.1)
    assert m.n_trees == 4
    for t in range(2):
        assert len(m.tree(t)["value"]) > 1
    for t in range(2, 4):
        assert len(m.tree(t)["value"]) == 1
