"""Oracle categorical splits pinned by the reference's own categorical tests
(tests/test_categorical.mojo, restated on their inputs) and by what the
mathematics fixes (Fisher's ordering: the best two-way partition of the
categories under the second-order score is a prefix of the g/h order, so the
two-direction walk must match a brute force over every subset).
"""
import itertools

import numpy as np
import pytest

import oracle_lib as O


def planes(grad, hess, count):
    gh = np.stack([np.asarray(grad, float), np.asarray(hess, float)], axis=1)
    return gh, np.asarray(count, np.int64)


def test_onehot_search_isolates_one_category():
    # test_categorical.mojo:210-234: three categories, one-vs-rest; only bin 2
    # has a positive gradient sum.
    gh, c = planes([0.0, -4.0, 8.0, -4.0], [0.0, 4.0, 4.0, 4.0], [0, 4, 4, 4])
    found, gain, left = O.cat_split(gh, c, 3, lambda_l2=0.0, min_data_in_leaf=0,
                                    max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=1.0,
                                    cat_l2=0.0, min_data_per_group=1)
    assert found and gain > 0.0
    assert left == [2]  # bin 0 (missing, unseen) is never a member


def test_sorted_search_groups_non_adjacent_categories():
    # test_categorical.mojo:236-267: bins 2, 4, 6 share one gradient sign,
    # bins 1, 3, 5 the other; max_cat_to_onehot=1 forces the sorted walk.
    grad = [0.0] + [-6.0 if b % 2 == 0 else 6.0 for b in range(1, 7)]
    gh, c = planes(grad, [0.0] + [6.0] * 6, [0] + [6] * 6)
    found, gain, left = O.cat_split(gh, c, 6, lambda_l2=0.0, min_data_in_leaf=0,
                                    max_cat_to_onehot=1, max_cat_threshold=32, cat_smooth=1.0,
                                    cat_l2=0.0, min_data_per_group=1)
    assert found
    assert left in ([2, 4, 6], [1, 3, 5])


def test_max_cat_threshold_caps_the_set_size():
    # test_categorical.mojo:269-297
    grad = [0.0] + [b - 10.5 for b in range(1, 21)]
    gh, c = planes(grad, [0.0] + [10.0] * 20, [0] + [10] * 20)
    found, _, left = O.cat_split(gh, c, 20, lambda_l2=0.0, min_data_in_leaf=0,
                                 max_cat_to_onehot=1, max_cat_threshold=3, cat_smooth=1.0,
                                 cat_l2=0.0, min_data_per_group=1)
    assert found and 1 <= len(left) <= 3


def test_onehot_boundary_counts_the_dummy_bin():
    # categorical.mojo:714-752: one-vs-rest while n_categories + 1 <=
    # max_cat_to_onehot (LightGBM's num_bin counts bin 0), so at the default
    # 4, three categories are one-hot and four take the sorted walk, whose
    # best set here holds two categories.
    gh, c = planes([0.0, 5.0, 5.0, -5.0, -5.0], [0.0, 5.0, 5.0, 5.0, 5.0], [0, 50, 50, 50, 50])
    kw = dict(lambda_l2=0.0, min_data_in_leaf=0, max_cat_to_onehot=4, cat_smooth=1.0, cat_l2=0.0,
              min_data_per_group=1)
    found, _, left = O.cat_split(gh, c, 4, **kw)
    assert found and len(left) == 2 and left in ([1, 2], [3, 4])
    found3, _, left3 = O.cat_split(gh[:4], c[:4], 3, **kw)
    assert found3 and len(left3) == 1


def brute_force_best(g, h, lam):
    """max over every proper nonempty subset S of the categories of
    G_S^2/(H_S+lam) + G_R^2/(H_R+lam) - G^2/(H+lam)."""
    n = len(g)
    G, H = g.sum(), h.sum()
    parent = G * G / (H + lam)
    best = -np.inf
    for k in range(1, n):
        for s in itertools.combinations(range(n), k):
            m = np.zeros(n, bool)
            m[list(s)] = True
            gl, hl = g[m].sum(), h[m].sum()
            best = max(best, gl * gl / (hl + lam) + (G - gl) ** 2 / (H - hl + lam) - parent)
    return best


@pytest.mark.parametrize("seed", range(12))
def test_sorted_walk_finds_the_best_partition(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(4, 10))
    g = rng.normal(size=n) * 10
    h = rng.uniform(1.0, 20.0, size=n)
    gh, c = planes(np.r_[0.0, g], np.r_[0.0, h], np.r_[0, np.full(n, 1000)])
    found, gain, left = O.cat_split(gh, c, n, lambda_l2=0.5, min_data_in_leaf=0,
                                    min_child_hess=0.0, max_cat_to_onehot=1,
                                    max_cat_threshold=64, cat_smooth=1e-12, cat_l2=0.0,
                                    min_data_per_group=1)
    want = brute_force_best(g, h, 0.5)
    assert found
    assert gain == pytest.approx(want, rel=1e-9, abs=1e-9)
    # the reported set scores the reported gain
    m = np.zeros(n, bool)
    m[[b - 1 for b in left]] = True
    G, H = g.sum(), h.sum()
    got = g[m].sum() ** 2 / (h[m].sum() + 0.5) + (G - g[m].sum()) ** 2 / (H - h[m].sum() + 0.5) \
        - G * G / (H + 0.5)
    assert got == pytest.approx(gain, rel=1e-9, abs=1e-9)


def test_min_data_per_group_and_smoothing_filter_categories():
    # cat_enters_search (tree_parameters_extra.mojo:1002-1006): a category
    # with fewer rows than cat_smooth never enters the walk; its rows stay
    # right. Category 3 alone would make the best set, but holds 5 rows.
    gh, c = planes([0.0, 4.0, -4.0, 50.0, -4.0], [0.0, 8.0, 8.0, 2.0, 8.0], [0, 40, 40, 5, 40])
    found, _, left = O.cat_split(gh, c, 4, lambda_l2=0.0, min_data_in_leaf=0,
                                 max_cat_to_onehot=1, cat_smooth=10.0, cat_l2=0.0,
                                 min_data_per_group=1)
    assert found and 3 not in left


def grouped(n_rows, n_cat):
    """test_categorical.mojo:315-324: the effect alternates with the code."""
    codes = np.arange(n_rows) % n_cat
    y = np.where(codes % 2 == 0, 1.0, -1.0)
    return codes, y


def small_cat(**kw):
    # CategoricalParams(4, 32, 2.0, 10.0, 5), test_categorical.mojo:68-73
    return dict(max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=2.0, cat_l2=10.0,
                min_data_per_group=5, **kw)


def fit_cat(codes, y, n_cat, num_leaves, n_trees, categorical=True):
    n = len(y)
    bins = (codes + 1).astype(np.uint8) if categorical else codes.astype(np.uint8)
    p, nc = O.categorical_params(
        [n_cat if categorical else 0], objective=O.OBJ_L2, num_iterations=n_trees,
        learning_rate=0.2, num_leaves=num_leaves, min_data_in_leaf=5, lambda_l2=1.0,
        min_sum_hessian=1e-3, **small_cat())
    m = O.train(bins, n, 1, 64, y, p)
    return m, bins


def test_low_cardinality_model_fits_the_grouping():
    # test_categorical.mojo:327-343
    codes, y = grouped(400, 4)
    m, _ = fit_cat(codes, y, 4, 8, 30)
    raw, _ = m.predict_binned(np.arange(1, 5, dtype=np.uint8), 4, 1)
    assert np.allclose(raw, [1.0, -1.0, 1.0, -1.0], atol=0.05)


def test_high_cardinality_beats_ordinal_treatment():
    # test_categorical.mojo:346-374
    codes, y = grouped(1000, 20)
    mc, bc = fit_cat(codes, y, 20, 4, 20)
    mn, bn = fit_cat(codes, y, 20, 4, 20, categorical=False)
    rc, _ = mc.predict_binned(bc, 1000, 1)
    rn, _ = mn.predict_binned(bn, 1000, 1)
    cat_sse = ((rc - y) ** 2).sum()
    num_sse = ((rn - y) ** 2).sum()
    assert cat_sse / 1000 < 0.02
    assert num_sse > 10.0 * cat_sse


def test_trees_record_categorical_splits_and_unknown_routes_right():
    # test_categorical.mojo:377-437
    codes, y = grouped(400, 6)
    m, bins = fit_cat(codes, y, 6, 4, 3)
    internal = m.feature >= 0
    assert internal.any()
    assert (m.threshold[internal] == -1).all()
    assert (m.missing_bin[internal] == -1).all()
    assert (m.default_left[internal] == 0).all()
    assert (m.cat_bits[internal].any(axis=1)).all()
    assert ((m.cat_bits[:, 0] & np.uint64(1)) == 0).all()  # bin 0 in no set
    # the unknown bin takes the right branch at every categorical node
    raw0, _ = m.predict_binned(np.zeros(1, np.uint8), 1, 1)
    want = np.float64(m.base[0])
    for t in range(m.n_trees):
        a = m.off[t]
        node = 0
        while m.feature[a + node] >= 0:
            node = m.right[a + node]
        want = want + 0.2 * m.value[a + node]
    assert raw0[0] == pytest.approx(want, rel=1e-12, abs=1e-15)


def test_quantized_categorical_training_runs_and_learns():
    codes, y = grouped(2000, 12)
    bins = (codes + 1).astype(np.uint8)
    p, nc = O.categorical_params([12], objective=O.OBJ_L2, num_iterations=20, learning_rate=0.2,
                                 num_leaves=8, min_data_in_leaf=5, use_quantized_grad=1,
                                 num_grad_quant_bins=16, **small_cat())
    m = O.train(bins, 2000, 1, 64, y, p)
    raw, _ = m.predict_binned(bins, 2000, 1)
    assert ((raw - y) ** 2).mean() < 0.05
    assert (m.threshold[m.feature >= 0] == -1).all()


def test_more_categories_than_bins_is_rejected():
    # test_categorical.mojo:196-207
    p, nc = O.categorical_params([64], objective=O.OBJ_L2, num_iterations=1)
    with pytest.raises(RuntimeError, match="more categories than bins"):
        O.train(np.zeros(10, np.uint8), 10, 1, 64, np.zeros(10), p)
