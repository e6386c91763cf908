"""GPU parity for categorical set splits (categorical.find_best_categorical_
split, src/mojotrees/categorical.mojo): device training against the CPU
oracle on the same bins -- trees, category sets, values and raw scores
bit-exact on the quantized path -- and the public surface end to end
(estimator with categorical_feature -> C ABI -> model with category tables ->
save/load -> host and device prediction).
"""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return device


def bits(a):
    return np.asarray(a, np.float64).view(np.uint64)


def cat_data(n, seed, cards=(3, 9, 40, 200), n_num=4):
    """n_num N(0,1) columns then one integer column per cardinality; the
    label mixes a numeric term with a random effect per category value, so
    both kinds of split win nodes."""
    rng = np.random.default_rng(seed)
    num = rng.normal(size=(n_num, n))
    cats = [rng.integers(0, c, size=n).astype(np.float64) for c in cards]
    z = num[0] - 0.5 * num[min(1, n_num - 1)] * num[n_num - 1]
    for j, c in enumerate(cards):
        eff = rng.normal(size=c) * (1.5 if j % 2 else 0.8)
        z = z + eff[cats[j].astype(int)]
    x = np.vstack([num] + cats)
    cat_idx = list(range(n_num, n_num + len(cards)))
    return x, z, cat_idx


def compare(fit, ref, n):
    assert fit.n_trees == ref.n_trees, (fit.n_trees, ref.n_trees)
    assert np.array_equal(fit.off, ref.off)
    for k in ("feature", "threshold", "left", "right", "default_left", "missing_bin"):
        assert np.array_equal(getattr(fit, k), getattr(ref, k)), k
    assert np.array_equal(fit.cat_bits, ref.cat_bits)
    for k in ("value", "gain", "count"):
        assert np.array_equal(bits(getattr(fit, k)), bits(getattr(ref, k))), k
    assert np.array_equal(bits(fit.train_raw()), bits(ref.train_raw(n)))


CAT = dict(max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=10.0, cat_l2=10.0,
           min_data_per_group=100)


@pytest.mark.parametrize("objective,leaves,trees", [(0, 31, 10), (1, 63, 8)])
def test_training_categorical_bit_exact(dev, objective, leaves, trees):
    n = 120_000
    x, z, cat_idx = cat_data(n, seed=3 + objective)
    rng = np.random.default_rng(7)
    y = z + 0.1 * rng.normal(size=n) if objective == 0 else \
        (rng.uniform(size=n) < 1 / (1 + np.exp(-z))).astype(np.float64)
    f = x.shape[0]
    bins, mb, nc = dev.bin_dense(x.ravel(), n, f, max_bins=255, categorical=cat_idx)
    assert nc.tolist() == [0, 0, 0, 0, 3, 9, 40, 200]
    kw = dict(objective=objective, num_iterations=trees, num_leaves=leaves, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    fit = dev.Dataset(bins, n, f, 255, y, missing_bin=mb, n_categories=nc).train(**kw, **CAT)
    p, keep = O.categorical_params(nc, **kw, **CAT, use_quantized_grad=1)
    ref = O.train(bins, n, f, 255, y, p, missing_bin=mb)
    cat_nodes = (fit.feature >= 0) & (fit.threshold < 0)
    assert cat_nodes.sum() > 0 and ((fit.feature >= 0) & (fit.threshold >= 0)).sum() > 0
    compare(fit, ref, n)
    # the device predictor routes the sets as the host one does
    raw, _ = ref.predict_binned(bins, n, f)
    assert np.array_equal(bits(fit.predict_binned(bins, n, f)), bits(raw))


def test_training_categorical_onehot_and_small_groups(dev):
    """One-vs-rest (3 categories <= max_cat_to_onehot - 1), a CatBoost
    one_hot_max_size override, and small min_data_per_group / cat_smooth so
    the sorted walk's guards and caps engage."""
    n = 40_000
    x, z, cat_idx = cat_data(n, seed=11, cards=(3, 6, 17), n_num=2)
    y = z + 0.2 * np.random.default_rng(1).normal(size=n)
    f = x.shape[0]
    bins, mb, nc = dev.bin_dense(x.ravel(), n, f, max_bins=63, categorical=cat_idx)
    for extra in (dict(max_cat_to_onehot=4, max_cat_threshold=3, cat_smooth=2.0, cat_l2=1.0,
                       min_data_per_group=5, one_hot_max_size=-1),
                  dict(max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=10.0, cat_l2=10.0,
                       min_data_per_group=50, one_hot_max_size=6)):
        kw = dict(objective=0, num_iterations=6, num_leaves=15, min_data_in_leaf=5, lambda_l2=1.0,
                  learning_rate=0.2)
        fit = dev.Dataset(bins, n, f, 63, y, missing_bin=mb, n_categories=nc).train(**kw, **extra)
        p, keep = O.categorical_params(nc, **kw, **extra, use_quantized_grad=1)
        ref = O.train(bins, n, f, 63, y, p, missing_bin=mb)
        compare(fit, ref, n)


def test_training_categorical_tied_keys_around_64_categories(dev):
    """Twin categories with equal sort keys, on both sides of the search's
    64-category boundary (below it a half's four waves rank bins 0-63
    together, from 64 on each lane ranks its own bin): rows come in pairs
    identical but for their category (c and c + 32), so with nearest
    rounding the twins' gradient sums, keys and counts are equal wherever
    both sit in one leaf, and the rank must keep the lower bin first."""
    m = 30_000
    rng = np.random.default_rng(21)
    num = np.repeat(rng.normal(size=(2, m)), 2, axis=1)          # twins share the numbers
    a = rng.integers(0, 32, size=m)
    b = rng.integers(0, 33, size=m)
    twin = np.arange(2 * m) % 2
    col64 = np.repeat(a, 2) + 32 * twin                           # 64 categories
    col65 = np.repeat(b, 2) + 32 * twin                           # 65 categories
    col63 = rng.integers(0, 63, size=2 * m)                       # 63 categories, no twins
    eff_a, eff_b = rng.normal(size=32), rng.normal(size=33)
    z = num[0] - 0.5 * num[1] + np.repeat(eff_a[a] + 0.7 * eff_b[b], 2)
    y = z + 0.1 * np.repeat(rng.normal(size=m), 2)
    x = np.vstack([num, col64, col65, col63]).astype(np.float64)
    n, f = 2 * m, x.shape[0]
    cat_idx = [2, 3, 4]
    bins, mb, nc = dev.bin_dense(x.ravel(), n, f, max_bins=255, categorical=cat_idx)
    assert nc.tolist() == [0, 0, 64, 65, 63]
    extra = dict(max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=5.0, cat_l2=1.0,
                 min_data_per_group=20)
    kw = dict(objective=0, num_iterations=5, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.2, stochastic_rounding=0)
    fit = dev.Dataset(bins, n, f, 255, y, missing_bin=mb, n_categories=nc).train(**kw, **extra)
    p, keep = O.categorical_params(nc, **kw, **extra, use_quantized_grad=1)
    ref = O.train(bins, n, f, 255, y, p, missing_bin=mb)
    assert ((fit.feature >= 2) & (fit.threshold < 0)).sum() > 0
    compare(fit, ref, n)


def test_training_categorical_fp32(dev):
    """fp32 gradients with fp64 histogram sums (the reference's own path):
    the sums differ from the oracle's only in rounding order, so the bar is
    the fp32 one -- the same splits and category sets, values within 1e-5
    relative, raw scores within 1e-5."""
    n = 80_000
    x, z, cat_idx = cat_data(n, seed=13, cards=(3, 12, 50))
    y = z + 0.1 * np.random.default_rng(3).normal(size=n)
    f = x.shape[0]
    bins, mb, nc = dev.bin_dense(x.ravel(), n, f, max_bins=255, categorical=cat_idx)
    kw = dict(objective=0, num_iterations=6, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    fit = dev.Dataset(bins, n, f, 255, y, missing_bin=mb, n_categories=nc).train(
        **kw, **CAT, use_quantized_grad=0)
    p, keep = O.categorical_params(nc, **kw, **CAT, use_quantized_grad=0)
    ref = O.train(bins, n, f, 255, y, p, missing_bin=mb)
    assert fit.n_trees == ref.n_trees
    for k in ("feature", "threshold", "left", "right", "default_left"):
        assert np.array_equal(getattr(fit, k), getattr(ref, k)), k
    assert np.array_equal(fit.cat_bits, ref.cat_bits)
    assert ((fit.feature >= 0) & (fit.threshold < 0)).sum() > 0
    assert np.allclose(fit.value, ref.value, rtol=1e-5, atol=1e-12)
    assert np.allclose(fit.train_raw(), ref.train_raw(n), rtol=1e-5, atol=1e-9)


def test_estimator_categorical_through_c_abi(dev, tmp_path):
    from mojoboost_amd.sklearn import MojoTreesRegressor

    n = 60_000
    x, z, cat_idx = cat_data(n, seed=5, cards=(7, 30))
    X = np.ascontiguousarray(x.T)
    X[np.random.default_rng(4).uniform(size=n) < 0.03, cat_idx[0]] = np.nan  # missing codes
    y = z + 0.1 * np.random.default_rng(9).normal(size=n)
    est = MojoTreesRegressor(n_estimators=8, num_leaves=31, max_bin=63, device="gpu",
                             use_quantized_grad=True, categorical_feature=cat_idx, min_data_per_group=50)
    est.fit(X, y)
    pred = est.predict(X)
    # the oracle on the library's own bins of the same matrix
    f = x.shape[0]
    bins, mb, nc = dev.bin_dense(np.ascontiguousarray(X.T).ravel(), n, f, max_bins=63, categorical=cat_idx)
    p, keep = O.categorical_params(nc, objective=0, num_iterations=8, num_leaves=31, learning_rate=0.1,
                                   min_data_in_leaf=20, lambda_l2=1.0, min_sum_hessian=1e-3,
                                   use_quantized_grad=1, max_cat_to_onehot=4, max_cat_threshold=32,
                                   cat_smooth=10.0, cat_l2=10.0, min_data_per_group=50)
    ref = O.train(bins, n, f, 63, y, p, missing_bin=mb)
    want, _ = ref.predict_binned(bins, n, f)
    assert np.array_equal(bits(pred), bits(want))
    # unseen codes predict like missing ones: right at every categorical node
    Xu = X[:100].copy()
    Xm = X[:100].copy()
    Xu[:, cat_idx[1]] = 1000.0
    Xm[:, cat_idx[1]] = np.nan
    assert np.array_equal(bits(est.predict(Xu)), bits(est.predict(Xm)))
    # the file keeps the category tables and sets; device prediction agrees
    path = tmp_path / "cat.txt"
    est.save(str(path))
    text = path.read_text()
    assert "\ncategorical 6 " in text and "\ncat " in text
    back = MojoTreesRegressor.load(str(path))
    assert np.array_equal(bits(back.predict(X)), bits(pred))
    assert np.array_equal(bits(back.predict(X, device="gpu")), bits(pred))
