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


# ---- multiclass GOSS (boosting._multiclass_goss_select, boosting.mojo:3680-3710,
# used once per round at :4041-4053)

def _probs(n, K, seed):
    rng = np.random.default_rng(seed)
    p = rng.dirichlet(np.ones(K) * 0.7, size=n)
    y = rng.integers(0, K, size=n).astype(np.float64)
    return p, y


def test_multiclass_sample_is_the_single_output_sample_of_the_class_sum():
    """The round's importance is the class sum, in class order, of
    |grad_k * hess_k| with each class's derivatives as its tree uses them
    (pinned: the golden softmax fits). The multiclass selection must then be
    goss_select over that importance: the single-output selection with
    grad = importance and hess = 1 (|importance * 1| is the importance
    itself), same rows, same weighted rows, same multiplier."""
    for K, seed in ((3, 1), (5, 2), (2, 3)):
        p, y = _probs(4000, K, seed)
        w = np.random.default_rng(seed).uniform(0.5, 2.0, size=len(y)) if K == 5 else None
        imp = np.zeros(len(y))
        for k in range(K):
            if w is None:
                g, h = O.grad_hess(O.OBJ_MULTICLASS, p.ravel(), y, num_class=K, class_k=k)
            else:
                g, h = O.grad_hess_w(O.OBJ_MULTICLASS, p.ravel(), y, w, num_class=K, class_k=k)
            imp += np.abs(g * h)
        rows, other, mult = O.goss_select_multiclass(p, y, K, 0.25, 0.15, seed=7, round_index=4, weights=w)
        srows, sscale, _, _ = O.goss_select(imp, np.ones(len(y)), 0.25, 0.15, 7, 4)
        assert np.array_equal(rows, srows)
        assert np.array_equal(np.flatnonzero(other), srows[sscale != 1.0])
        assert np.all(sscale[sscale != 1.0] == mult)


def test_multiclass_importance_counts_every_class():
    """A row whose true class is badly predicted in one class only must
    outrank rows that every class predicts well: dropping a class from the
    sum (or taking one class's term) changes which rows are on top."""
    n, K = 1000, 4
    p = np.full((n, K), 0.25)
    y = np.zeros(n)
    # rows 0..99: class 3 confidently wrong (label 3, p_3 small)
    p[:100] = [0.7, 0.1, 0.1, 0.1]
    y[:100] = 3
    # rows 100..: well predicted (label 0, p_0 large)
    p[100:] = [0.97, 0.01, 0.01, 0.01]
    rows, other, _ = O.goss_select_multiclass(p, y, K, 0.1, 0.0, seed=1, round_index=0)
    assert np.array_equal(rows, np.arange(100))
    assert not other.any()


def test_multiclass_goss_with_every_row_on_top_trains_like_no_goss():
    """top_rate = 1 puts every row on top with weight 1: past the warmup the
    rounds train on every row, so the fit equals a fit without GOSS, tree for
    tree (quantized and fp32)."""
    n, f, K = 3000, 4, 3
    rng = np.random.default_rng(5)
    x = rng.normal(size=(f, n))
    y = np.argmax(x[:K] + 0.3 * rng.normal(size=(K, n)), axis=0).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=32)
    for quantized in (1, 0):
        kw = dict(objective=O.OBJ_MULTICLASS, num_class=K, num_iterations=6, num_leaves=15,
                  learning_rate=0.5, use_quantized_grad=quantized)
        plain = O.train(bins, n, f, 32, y, O.default_params(**kw), missing_bin=mb)
        goss = O.train(bins, n, f, 32, y, O.default_params(**kw, goss=1, top_rate=1.0, other_rate=0.0),
                       missing_bin=mb)
        assert plain.n_trees == goss.n_trees == 6 * K
        for t in range(plain.n_trees):
            a, b = plain.tree(t), goss.tree(t)
            assert np.array_equal(a["feature"], b["feature"]) and np.array_equal(a["threshold"], b["threshold"])
            assert np.array_equal(a["value"].view(np.uint64), b["value"].view(np.uint64))


def test_multiclass_goss_samples_after_warmup():
    n, f, K = 4000, 4, 3
    rng = np.random.default_rng(6)
    x = rng.normal(size=(f, n))
    y = np.argmax(x[:K] + 0.3 * rng.normal(size=(K, n)), axis=0).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=32)
    kw = dict(objective=O.OBJ_MULTICLASS, num_class=K, num_iterations=5, num_leaves=7,
              learning_rate=0.5, use_quantized_grad=1, min_data_in_leaf=5)
    m = O.train(bins, n, f, 32, y, O.default_params(**kw, goss=1, top_rate=0.2, other_rate=0.1), missing_bin=mb)
    # warmup floor(1 / 0.5) = 2 rounds on every row, then one sample per
    # round of at least 0.2 n + 0.1 n rows (rows tied with the top_k-th
    # importance all stay on top): every class tree of a round has it as
    # its root count
    roots = np.array([m.tree(t)["count"][0] for t in range(m.n_trees)]).reshape(-1, K)
    assert np.all(roots[:2] == n)
    assert np.all(roots[2:] >= 0.3 * n) and np.all(roots[2:] < n)
    assert np.all(roots[2:] == roots[2:, :1])
