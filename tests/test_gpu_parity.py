"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

Bar: quantized-gradient histograms, split
choices, trees and raw scores bit-exact. Every comparison below is on
integers or on IEEE-754 bit patterns.
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


def c2_like(n, f=28, seed=1, nb=255):
    """C2-shaped data at a reduced row count:
    21 N(0,1) columns, 7 derived (products and abs of pairs), label
    Bernoulli(sigmoid(sum of 8 pairwise terms))."""
    rng = np.random.default_rng(seed)
    base = rng.normal(size=(21, n))
    derived = [base[0] * base[1], np.abs(base[2]), base[3] * base[4], np.abs(base[5] * base[6]),
               base[7] * base[8], np.abs(base[9]) * base[10], base[11] * base[12]]
    x = np.vstack([base] + derived)[:f]
    pairs = rng.integers(0, 21, size=(8, 2))
    w = rng.uniform(-1, 1, size=8)
    logit = 0.3 + sum(w[i] * base[a] * base[b] for i, (a, b) in enumerate(pairs))
    y = (rng.uniform(size=n) < 1 / (1 + np.exp(-logit))).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=nb)
    return bins, y, mb, nb


def test_exp_sigmoid_bit_exact(dev):
    L = O.lib()
    x = np.concatenate([np.linspace(-750, 750, 30001), np.random.default_rng(3).normal(0, 5, 20000),
                        [0.0, -0.0, 1e-300, -1e-300, 709.0, -709.5, 745.0]])
    e, s = dev.exp_sigmoid(x)
    want_e = np.array([L.orc_exp(float(v)) for v in x])
    want_s = np.array([L.orc_sigmoid(float(v)) for v in x])
    assert np.array_equal(bits(e), bits(want_e))
    assert np.array_equal(bits(s), bits(want_s))


@pytest.mark.parametrize("objective", [0, 1])
def test_objective_and_quantizer_bit_exact(dev, objective):
    n, f = 50_000, 6
    rng = np.random.default_rng(7 + objective)
    bins = rng.integers(0, 32, size=(f, n), dtype=np.uint8)
    y = (rng.uniform(size=n) < 0.4).astype(np.float64) if objective == 1 else rng.normal(size=n)
    raw = rng.normal(0, 2, size=n)
    ds = dev.Dataset(bins, n, f, 32, y)
    for rnd in (0, 5):
        g, h, qg, qh, sc = ds.objective_quantize(raw, round_index=rnd, objective=objective)
        og, oh = O.grad_hess(objective, raw, y)
        assert np.array_equal(g.astype(np.float64), og)
        assert np.array_equal(h.astype(np.float64), oh)
        oqg, oqh, osc = O.quantize(og, oh, quant_bins=4, stochastic=1, seed=11, round_index=rnd,
                                   const_hessian=1 if objective == 0 else 0)
        assert sc[0] == osc[0] and sc[1] == osc[1]
        assert np.array_equal(qg, oqg)
        assert np.array_equal(qh, oqh)


@pytest.mark.parametrize("subset", [False, True])
def test_histogram_bit_exact(dev, subset):
    n, f, nb = 300_000, 28, 255
    rng = np.random.default_rng(11)
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    bins[3] = bins[3] % 7          # a low-cardinality feature: hot bins
    qg = rng.integers(-2, 3, size=n).astype(np.int8)
    qh = rng.integers(0, 5, size=n).astype(np.int8)
    ds = dev.Dataset(bins, n, f, nb, np.zeros(n))
    rows = np.sort(rng.choice(n, 77_777, replace=False)).astype(np.int32) if subset else None
    got = ds.histogram(qg, qh, rows, quant_bins=4)
    want = O.hist_quantized(bins.ravel(), n, f, nb, qg, qh, rows)
    assert np.array_equal(got.astype(np.int64), want)


def _compare_fit(fit, ref, n):
    assert fit.n_trees == ref.n_trees, (fit.n_trees, ref.n_trees)
    assert np.array_equal(fit.off, ref.off)
    for k in ("feature", "threshold", "left", "right", "default_left", "missing_bin"):
        assert np.array_equal(getattr(fit, k), getattr(ref, k)), k
    for k in ("value", "gain", "count"):
        assert np.array_equal(bits(getattr(fit, k)), bits(getattr(ref, k))), k
    assert np.array_equal(bits(fit.base), bits(ref.base))
    assert np.array_equal(bits(fit.train_raw()), bits(ref.train_raw(n)))


def test_training_c2_shape_bit_exact(dev):
    """C2 workload shape (255 bins, 255 leaves, logistic, int8 g/h) at
    200k rows x 28 features, 12 trees: every tree and raw score identical."""
    n = 200_000
    bins, y, mb, nb = c2_like(n)
    kw = dict(objective=1, num_iterations=12, num_leaves=255, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb)
    fit = ds.train(**kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_training_regression_const_hessian(dev):
    n, f, nb = 60_000, 10, 63
    rng = np.random.default_rng(21)
    x = rng.normal(size=(f, n))
    y = x[0] - 2 * x[1] * x[2] + 0.1 * rng.normal(size=n)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=nb)
    kw = dict(objective=0, num_iterations=8, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1, max_depth=6)
    fit = dev.Dataset(bins, n, f, nb, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_training_bagging_and_feature_fraction(dev):
    n = 50_000
    bins, y, mb, nb = c2_like(n, f=20, seed=5, nb=63)
    kw = dict(objective=1, num_iterations=6, num_leaves=63, min_data_in_leaf=10, lambda_l2=0.5,
              learning_rate=0.2, bagging_fraction=0.7, bagging_freq=2, bagging_seed=9,
              feature_fraction=0.6, feature_fraction_seed=4)
    fit = dev.Dataset(bins, n, 20, nb, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, 20, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_training_missing_values_and_tiny_leaves(dev):
    """NaNs reserve a missing bin: both routing directions are scanned."""
    n, f = 20_000, 5
    rng = np.random.default_rng(33)
    x = rng.normal(size=(f, n))
    x[1, rng.uniform(size=n) < 0.2] = np.nan
    x[3, rng.uniform(size=n) < 0.05] = np.nan
    y = (np.nan_to_num(x[1], nan=1.5) + x[0] > 0.3).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=32)
    assert (mb >= 0).sum() == 2
    kw = dict(objective=1, num_iterations=5, num_leaves=127, min_data_in_leaf=2, lambda_l2=0.0,
              min_sum_hessian=1e-3, learning_rate=0.3)
    fit = dev.Dataset(bins, n, f, 32, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, f, 32, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_training_is_deterministic(dev):
    n = 100_000
    bins, y, mb, nb = c2_like(n, seed=8)
    ds = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb)
    kw = dict(objective=1, num_iterations=4, num_leaves=255)
    a, b = ds.train(**kw), ds.train(**kw)
    for k in ("feature", "threshold", "value", "gain"):
        assert np.array_equal(getattr(a, k), getattr(b, k))
    assert np.array_equal(bits(a.train_raw()), bits(b.train_raw()))


@pytest.mark.parametrize("objective", ["binary", "regression"])
def test_estimator_through_c_abi_bit_exact(dev, tmp_path, objective):
    """The public surface end to end: MojoTrees*(device="gpu").fit ->
    mojotrees_train_dense -> host binning -> device training -> model ->
    predict, against the oracle trained on the oracle's own bins of the same
    matrix (identical bin boundaries); then save -> load -> predict."""
    from mojoboost_amd.sklearn import MojoTreesClassifier, MojoTreesRegressor

    n, f = 60_000, 8
    rng = np.random.default_rng(11)
    X = rng.normal(size=(n, f))
    X[rng.uniform(size=(n, f)) < 0.02] = np.nan
    z = X[:, 0] * X[:, 1] + np.abs(np.nan_to_num(X[:, 2])) - 0.5
    z = np.nan_to_num(z)
    if objective == "binary":
        y = (rng.uniform(size=n) < 1 / (1 + np.exp(-z))).astype(np.float64)
        est = MojoTreesClassifier(n_estimators=6, num_leaves=31, learning_rate=0.1,
                                  max_bin=63, device="gpu", use_quantized_grad=True)
    else:
        y = z + 0.1 * rng.normal(size=n)
        est = MojoTreesRegressor(n_estimators=6, num_leaves=31, learning_rate=0.1,
                                 max_bin=63, device="gpu", use_quantized_grad=True)
    est.fit(X, y)
    raw = est.decision_function(X) if objective == "binary" else est.predict(X)

    x_cm = np.ascontiguousarray(X.T).ravel()
    bins, _, _, mb = O.fit_transform(x_cm, n, f, max_bins=63)
    p = O.default_params(objective=1 if objective == "binary" else 0, num_iterations=6,
                         num_leaves=31, learning_rate=0.1, min_data_in_leaf=20, lambda_l2=1.0,
                         min_sum_hessian=1e-3, use_quantized_grad=1, num_grad_quant_bins=4,
                         stochastic_rounding=1)
    ref = O.train(bins, n, f, 64, y, p, missing_bin=mb)
    want_raw, _ = ref.predict_binned(bins, n, f)
    assert np.array_equal(bits(raw), bits(want_raw))

    path = tmp_path / "m.txt"
    est.save(str(path))
    back = type(est).load(str(path))
    raw2 = back.decision_function(X) if objective == "binary" else back.predict(X)
    assert np.array_equal(bits(raw2), bits(raw))


def c5_like(n, n_class=5, seed=5, nb=255):
    """C5-shaped data at reduced size: 16
    continuous N(0,1) columns and 4 integer columns of cardinality 4-64, the
    class drawn as the argmax of random linear scores plus Gumbel noise."""
    rng = np.random.default_rng(seed)
    cont = rng.normal(size=(16, n))
    cats = np.vstack([rng.integers(0, c, size=n) for c in (4, 9, 27, 64)]).astype(np.float64)
    x = np.vstack([cont, cats])
    w = rng.normal(size=(n_class, x.shape[0]))
    scores = w @ (x - x.mean(axis=1, keepdims=True)) / 4 + rng.gumbel(size=(n_class, n))
    y = scores.argmax(axis=0).astype(np.float64)
    f = x.shape[0]
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=nb)
    return bins, y, mb, nb, f


@pytest.mark.parametrize("bagging", [False, True])
def test_training_multiclass_bit_exact(dev, bagging):
    """Softmax multiclass, one tree per class per round, quantized per class:
    every tree and every training score identical to the oracle."""
    n, K = 120_000, 5
    bins, y, mb, nb, f = c5_like(n, K)
    kw = dict(objective=2, num_class=K, num_iterations=4, num_leaves=63, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    if bagging:
        kw.update(bagging_fraction=0.7, bagging_freq=1, bagging_seed=9)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    fit = ds.train(**kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    assert fit.num_class == K and fit.n_trees == 4 * K
    _compare_fit(fit, ref, n)


@pytest.mark.parametrize("K,bagging", [(2, False), (7, True)])
def test_training_multiclass_side_by_side_states(dev, K, bagging):
    """A round's class trees are grown by up to three states side by side,
    each on its own stream: two states for two classes, three for seven
    (growing classes 0, 3, 6 / 1, 4 / 2, 5). The oracle grows the classes in
    turn; every tree and training score must be identical."""
    n = 60_000
    bins, y, mb, nb, f = c5_like(n, K, seed=11)
    kw = dict(objective=2, num_class=K, num_iterations=3, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    if bagging:
        kw.update(bagging_fraction=0.6, bagging_freq=1, bagging_seed=4)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    fit = ds.train(**kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    assert fit.num_class == K and fit.n_trees == 3 * K
    _compare_fit(fit, ref, n)


def test_estimator_multiclass_through_c_abi_bit_exact(dev, tmp_path):
    """MojoTreesClassifier with 4 classes -> objective=multiclass through the
    C ABI; raw scores equal the oracle's on its own bins, and survive
    save -> load."""
    from mojoboost_amd.sklearn import MojoTreesClassifier

    n, f, K = 50_000, 6, 4
    rng = np.random.default_rng(21)
    X = rng.normal(size=(n, f))
    scores = X[:, :K] * 1.5 + rng.gumbel(size=(n, K))
    y = np.array(["a", "b", "c", "d"])[scores.argmax(axis=1)]
    est = MojoTreesClassifier(n_estimators=3, num_leaves=15, learning_rate=0.2, max_bin=63,
                              device="gpu", use_quantized_grad=True).fit(X, y)
    raw = est.decision_function(X)
    assert raw.shape == (n, K) and list(est.classes_) == ["a", "b", "c", "d"]

    x_cm = np.ascontiguousarray(X.T).ravel()
    bins, _, _, mb = O.fit_transform(x_cm, n, f, max_bins=63)
    yi = np.unique(y, return_inverse=True)[1].astype(np.float64)
    p = O.default_params(objective=2, num_class=K, num_iterations=3, num_leaves=15,
                         learning_rate=0.2, min_data_in_leaf=20, lambda_l2=1.0,
                         min_sum_hessian=1e-3, use_quantized_grad=1, num_grad_quant_bins=4,
                         stochastic_rounding=1)
    ref = O.train(bins, n, f, 64, yi, p, missing_bin=mb)
    want_raw, want_prob = ref.predict_binned(bins, n, f)
    assert np.array_equal(bits(raw.ravel()), bits(want_raw))
    prob = est.predict_proba(X)
    assert np.allclose(prob.ravel(), want_prob, rtol=1e-12, atol=0)

    path = tmp_path / "mc.txt"
    est.save(str(path))
    back = MojoTreesClassifier.load(str(path))
    assert np.array_equal(bits(back.decision_function(X).ravel()), bits(raw.ravel()))


def test_stop_rule_constant_labels(dev):
    """A round that cannot split and whose leaf value is below 1e-12 ends
    training (boosting._boost_rounds): no trees, scores stay at the base."""
    n = 20_000
    rng = np.random.default_rng(4)
    bins = rng.integers(0, 16, size=(3, n), dtype=np.uint8)
    y = np.full(n, 2.5)
    kw = dict(objective=0, num_iterations=5, num_leaves=15, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    ds = dev.Dataset(bins.ravel(), n, 3, 16, y)
    fit = ds.train(**kw)
    ref = O.train(bins.ravel(), n, 3, 16, y, O.default_params(**kw, use_quantized_grad=1))
    assert fit.n_trees == ref.n_trees == 0
    assert np.array_equal(bits(fit.train_raw()), bits(ref.train_raw(n)))


# ---------------------------------------------------------------- fp32 path
# Bar: fp32 histograms within 1e-5 relative of
# the reference's Float64 histograms, predictions after 100 trees within 1e-5
# relative. The device sums the fp32 gradient values in fp64 with atomics, so
# only the order (and with it the last bits) of the additions differs.

def test_histogram_fp32_matches_oracle(dev):
    n, f, nb = 300_000, 20, 64
    rng = np.random.default_rng(31)
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.01, 1.0, size=n).astype(np.float32)
    ds = dev.Dataset(bins.ravel(), n, f, nb, np.zeros(n))
    L = O.lib()
    for rows in (None, np.sort(rng.choice(n, size=n // 3, replace=False)).astype(np.int32)):
        gh, cnt = ds.histogram_fp32(g, h, rows)
        want_gh = np.zeros(2 * f * nb)
        want_c = np.zeros(f * nb, np.int64)
        r = None if rows is None else rows
        L.orc_hist_float(O._ptr(bins.ravel()), n, f, nb, O._ptr(g.astype(np.float64)),
                         O._ptr(h.astype(np.float64)), O._ptr(r), 0 if r is None else len(r), 1,
                         O._ptr(want_gh), O._ptr(want_c))
        assert np.array_equal(cnt, want_c)
        # per cell, the rounding of a different summation order is bounded by
        # n_cell * eps * sum |x|; 1e-12 of the cell's magnitude is far inside
        # the 1e-5 bar
        scale = np.maximum(np.abs(want_gh), 1e-30)
        rel = np.abs(gh - want_gh) / scale
        assert rel.max() < 1e-10, rel.max()


def _rel_err(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-12)))


def _tree_agreement(fit, ref):
    same = 0
    for t in range(min(fit.n_trees, ref.n_trees)):
        a, b = fit.tree(t), ref.tree(t)
        same += int(all(np.array_equal(a[k], b[k]) for k in ("feature", "threshold", "left", "right")))
    return same


def test_training_fp32_c1(dev):
    """C1 (the reference's CPU-runnable case):
    100k x 28 N(0,1), y = x.w + 0.1 N(0,1), L2, 255 bins, 31 leaves, lr 0.1,
    100 trees, fp32 gradients."""
    n, f = 100_000, 28
    rng = np.random.default_rng(0x5EED0001)
    x = rng.normal(size=(f, n)).astype(np.float32).astype(np.float64)
    w = rng.uniform(-1.0, 1.0, size=f)
    y = w @ x + 0.1 * rng.normal(size=n)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=255)
    kw = dict(objective=0, num_iterations=100, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, f, 255, y, missing_bin=mb)
    fit = ds.train(use_quantized_grad=0, **kw)
    ref = O.train(bins, n, f, 255, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=mb)
    assert fit.n_trees == ref.n_trees == 100
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    raw, _ = ref.predict_binned(bins, n, f)
    assert _rel_err(fit.train_raw(), raw) < 1e-5
    assert _tree_agreement(fit, ref) >= 95


@pytest.mark.parametrize("nb", [5, 13, 64])
def test_training_fp32_few_bins(dev, nb):
    """fp32 path at bin counts that take the scan's short paths: fewer than
    eight cells (no full eight-cell block: the totals are the remainder's
    sequential sum), one full block and a remainder, and whole blocks only;
    the same splits as the oracle, raw scores within 1e-5."""
    n, f = 40_000, 8
    bins, y, mb, nbb = c2_like(n, f=f, seed=31 + nb, nb=nb)
    kw = dict(objective=1, num_iterations=8, num_leaves=15, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.2)
    fit = dev.Dataset(bins, n, f, nbb, y, missing_bin=mb).train(use_quantized_grad=0, **kw)
    ref = O.train(bins, n, f, nbb, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=mb)
    assert fit.n_trees == ref.n_trees
    assert _tree_agreement(fit, ref) >= ref.n_trees - 1
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5


def test_training_fp32_binary_bagging(dev):
    n = 150_000
    bins, y, mb, nb = c2_like(n, f=16)
    kw = dict(objective=1, num_iterations=20, num_leaves=63, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1, bagging_fraction=0.8, bagging_freq=1, bagging_seed=5)
    ds = dev.Dataset(bins, n, 16, nb, y, missing_bin=mb)
    fit = ds.train(use_quantized_grad=0, **kw)
    ref = O.train(bins, n, 16, nb, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=mb)
    assert fit.n_trees == ref.n_trees
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(fit, ref) >= ref.n_trees - 1


@pytest.mark.parametrize("n,f,leaves,lr,iters", [(3_000, 4, 15, 0.2, 20), (200_000, 16, 63, 0.1, 16)])
def test_training_goss_fp32(dev, n, f, leaves, lr, iters):
    """GOSS (goss.mojo:294-396) on the fp32 path, as in C3: warmup of
    floor(1/lr) rounds, then the top 20 % by |g h| plus selection sampling of
    10 % weighted by (n - top_k) / other_k. The sample is exact (the small
    case makes the sampling's one-by-one steps frequent), so the trees follow
    the oracle's and predictions agree within 1e-5."""
    bins, y, mb, nb = c2_like(n, f=f, seed=13)
    kw = dict(objective=1, num_iterations=iters, num_leaves=leaves, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=lr)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    fit = ds.train(use_quantized_grad=0, goss=1, top_rate=0.2, other_rate=0.1, **kw)
    ref = O.train(bins, n, f, nb, y,
                  O.default_params(**kw, use_quantized_grad=0, goss=1, top_rate=0.2, other_rate=0.1),
                  missing_bin=mb)
    assert fit.n_trees == ref.n_trees
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(fit, ref) >= ref.n_trees - 1


# ------------------------------------------------------------ wide (C4-shaped)
def c4_like(n, f, seed=17, nb=63):
    """C4-shaped data at a reduced size: N(0,1)
    features, label = sign of a sparse 50-feature linear model plus noise."""
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(f, n))
    k = min(50, f)
    idx = rng.choice(f, k, replace=False)
    w = rng.normal(size=k)
    y = ((w @ x[idx] + 0.5 * rng.normal(size=n)) > 0).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=nb)
    return bins, y, mb, nb


@pytest.mark.parametrize("subset", [False, True])
def test_histogram_wide_bit_exact(dev, subset):
    """700 features at 63 bins: six feature tiles of 117 features, every
    (feature, bin) cell identical to the oracle's."""
    n, f, nb = 40_000, 700, 63
    rng = np.random.default_rng(12)
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    bins[699] = bins[699] % 3
    qg = rng.integers(-2, 3, size=n).astype(np.int8)
    qh = rng.integers(0, 5, size=n).astype(np.int8)
    ds = dev.Dataset(bins, n, f, nb, np.zeros(n))
    rows = np.sort(rng.choice(n, 9_999, replace=False)).astype(np.int32) if subset else None
    got = ds.histogram(qg, qh, rows, quant_bins=4)
    want = O.hist_quantized(bins.ravel(), n, f, nb, qg, qh, rows)
    assert np.array_equal(got.astype(np.int64), want)


def test_histogram_fp32_wide(dev):
    """fp32 histograms at 255 bins take 20 bytes per LDS cell, so 300
    features run as ten tiles of 30."""
    n, f, nb = 30_000, 300, 255
    rng = np.random.default_rng(13)
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.01, 1.0, size=n).astype(np.float32)
    ds = dev.Dataset(bins.ravel(), n, f, nb, np.zeros(n))
    gh, cnt = ds.histogram_fp32(g, h)
    want_gh = np.zeros(2 * f * nb)
    want_c = np.zeros(f * nb, np.int64)
    O.lib().orc_hist_float(O._ptr(bins.ravel()), n, f, nb, O._ptr(g.astype(np.float64)),
                           O._ptr(h.astype(np.float64)), None, 0, 1, O._ptr(want_gh), O._ptr(want_c))
    assert np.array_equal(cnt, want_c)
    rel = np.abs(gh - want_gh) / np.maximum(np.abs(want_gh), 1e-30)
    assert rel.max() < 1e-10, rel.max()


def test_training_c4_shape_bit_exact(dev):
    """C4 workload shape (2000 features, 63 bins, 127 leaves, logistic, int8
    g/h) at 20k rows, 3 trees: sixteen feature tiles; every tree and raw score
    identical to the oracle's."""
    n, f = 20_000, 2000
    bins, y, mb, nb = c4_like(n, f)
    kw = dict(objective=1, num_iterations=3, num_leaves=127, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    fit = ds.train(use_quantized_grad=1, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_training_wide_fp32_and_narrow_after_wide(dev):
    """fp32 gradients on 300 features at 255 bins (ten tiles) within 1e-5 of
    the oracle; then the same dataset trains quantized (the records are
    rebuilt for the other tile width) bit-exactly."""
    n, f = 30_000, 300
    bins, y, mb, nb = c4_like(n, f, seed=19, nb=255)
    kw = dict(objective=1, num_iterations=6, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    fit = ds.train(use_quantized_grad=0, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=mb)
    assert fit.n_trees == ref.n_trees
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(fit, ref) >= ref.n_trees - 1
    fitq = ds.train(use_quantized_grad=1, **kw)
    refq = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fitq, refq, n)


def test_goss_count_paths_agree(dev):
    """The GOSS count three ways: the default band (parallel decisions, a
    sequential count over the open rows, the exact check), the full
    sequential count alone, and a band so wrong that the check fails and the
    full count runs. All three give the same sample, hence bit-identical
    training, and the oracle's trees."""
    n, f = 200_000, 16
    bins, y, mb, nb = c2_like(n, f=f, seed=23)
    kw = dict(objective=1, num_iterations=14, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    goss = dict(use_quantized_grad=0, goss=1, top_rate=0.2, other_rate=0.1)
    a = ds.train(**goss, **kw)
    b = ds.train(**goss, goss_exact_walk=1, **kw)
    c = ds.train(**goss, goss_band=-1e9, **kw)
    for other in (b, c):
        assert np.array_equal(bits(a.train_raw()), bits(other.train_raw()))
        assert np.array_equal(a.threshold, other.threshold)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, **goss), missing_bin=mb)
    assert a.n_trees == ref.n_trees
    assert _rel_err(a.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(a, ref) >= ref.n_trees - 1


# ------------------------------------------------------------- prediction
def test_device_predict_bit_exact(dev):
    """Device prediction (mbh_predict_binned) of a trained ensemble: the raw
    scores of the training rows equal the trainer's own (same fused updates in
    the same order) and the oracle's host predictor, bit for bit; an
    iteration range without tree 0 leaves the base score out."""
    n = 120_000
    bins, y, mb, nb = c2_like(n, f=20, seed=29, nb=63)
    kw = dict(objective=1, num_iterations=20, num_leaves=63, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    fit = dev.Dataset(bins, n, 20, nb, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, 20, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    raw = fit.predict_binned(bins, n, 20)
    assert np.array_equal(bits(raw), bits(fit.train_raw()))
    want, _ = ref.predict_binned(bins, n, 20)
    assert np.array_equal(bits(raw), bits(want))
    tail = fit.predict_binned(bins, n, 20, tree_begin=5)
    head = fit.predict_binned(bins, n, 20, tree_begin=0, tree_end=5)
    assert np.allclose(head + tail, raw, rtol=1e-12, atol=1e-12)


def test_device_predict_wide_multiclass_through_c_abi(dev):
    """mojotrees_predict_ex with device=GPU against device=CPU: multiclass
    softmax and a 300-feature model (feature tiles), raw and response,
    whole ensemble and iteration slices -- identical bits."""
    from mojoboost_amd.sklearn import MojoTreesClassifier

    rng = np.random.default_rng(31)
    for n, f, k in ((40_000, 12, 4), (20_000, 300, 2)):
        X = rng.normal(size=(n, f))
        X[rng.uniform(size=(n, f)) < 0.01] = np.nan
        score = np.nan_to_num(X[:, :k]) + 0.5 * rng.normal(size=(n, k))
        y = np.argmax(score, axis=1)
        est = MojoTreesClassifier(n_estimators=8, num_leaves=15, learning_rate=0.2, max_bin=63,
                                  device="gpu", use_quantized_grad=True).fit(X, y)
        for s0, num in ((0, None), (3, None), (0, 5), (2, 3)):
            a = est.decision_function(X, start_iteration=s0, num_iteration=num)
            b = est.decision_function(X, start_iteration=s0, num_iteration=num, device="gpu")
            assert np.array_equal(bits(a), bits(b)), (n, f, s0, num)
            pa = est.predict_proba(X, start_iteration=s0, num_iteration=num)
            pb = est.predict_proba(X, start_iteration=s0, num_iteration=num, device="gpu")
            assert np.array_equal(bits(pa), bits(pb)), (n, f, s0, num)
        assert np.array_equal(est.predict(X, device="auto"), est.predict(X))


# --------------------------------------------------------------- lambdarank
def ranking_data(n_queries, f=10, seed=41, max_q=200, grades=4):
    """Queries of 1..max_q documents; the relevance grade follows a noisy
    linear score of the features."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(1, max_q + 1, size=n_queries)
    n = int(counts.sum())
    x = rng.normal(size=(f, n))
    s = x[0] - 0.5 * x[1] + 0.3 * x[2] * x[3] + 0.5 * rng.normal(size=n)
    y = np.clip(np.floor((s + 2.0) * grades / 4.0), 0, grades).astype(np.float64)
    return x, y, counts.astype(np.int32), n


@pytest.mark.parametrize("trunc,norm", [(30, True), (5, True), (30, False), (1, True)])
def test_lambdarank_gradients_bit_exact(dev, trunc, norm):
    """The device lambdas (ranking._fill_query_lambdas in binary64): every
    gradient and hessian bit equal to the oracle's, over queries of 1 to
    2048 documents with tied scores and grades up to 30."""
    rng = np.random.default_rng(43 + trunc)
    counts = np.array([1, 2, 3, 7, 64, 65, 300, 2048, 1, 129, 5], np.int32)
    n = int(counts.sum())
    y = rng.integers(0, 5, size=n).astype(np.float64)
    y[:40] = rng.integers(0, 31, size=40)
    raw = np.round(rng.normal(size=n), 1)             # many ties
    raw[100:140] = 0.0
    bins = rng.integers(0, 8, size=(2, n), dtype=np.uint8)
    ds = dev.Dataset(bins, n, 2, 8, y)
    ds.set_groups(counts)
    g, h = ds.lambdarank(raw, lambdarank_truncation_level=trunc, lambdarank_norm=int(norm))
    wg, wh = O.lambdarank(raw, y, counts, truncation=trunc, sigma=1.0, norm=norm)
    assert np.array_equal(bits(g), bits(wg))
    assert np.array_equal(bits(h), bits(wh))


@pytest.mark.parametrize("trunc,norm", [(30, True), (5, False)])
def test_lambdarank_large_queries_bit_exact(dev, trunc, norm):
    """Queries above the LDS sort's 2048 documents (one of 10000) are sorted
    and paired in global memory, their pair values staged in LDS chunks:
    every gradient and hessian bit still equal to the oracle's, beside small
    queries in the same launch."""
    rng = np.random.default_rng(71 + trunc)
    counts = np.array([10_000, 3, 2049, 4097, 700, 2048, 1, 2050], np.int32)
    n = int(counts.sum())
    y = rng.integers(0, 5, size=n).astype(np.float64)
    y[5000:5100] = rng.integers(0, 31, size=100)
    raw = np.round(rng.normal(size=n), 1)             # many ties
    raw[9000:9500] = 0.0
    bins = rng.integers(0, 8, size=(2, n), dtype=np.uint8)
    ds = dev.Dataset(bins, n, 2, 8, y)
    ds.set_groups(counts)
    g, h = ds.lambdarank(raw, lambdarank_truncation_level=trunc, lambdarank_norm=int(norm))
    wg, wh = O.lambdarank(raw, y, counts, truncation=trunc, sigma=1.0, norm=norm)
    assert np.array_equal(bits(g), bits(wg))
    assert np.array_equal(bits(h), bits(wh))


def test_training_lambdarank_large_queries(dev):
    """A quantized LambdaRank fit whose queries include three above 2048
    documents: every tree and raw score bit-exact to the oracle."""
    rng = np.random.default_rng(77)
    counts = np.concatenate([[3000, 5000, 2500], rng.integers(1, 200, size=60)]).astype(np.int32)
    n = int(counts.sum())
    x = rng.normal(size=(10, n))
    sc = x[0] - 0.5 * x[1] + 0.3 * x[2] * x[3] + 0.5 * rng.normal(size=n)
    y = np.clip(np.floor((sc + 2.0)), 0, 4).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, 10, max_bins=63)
    kw = dict(num_iterations=5, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, 10, 64, y, missing_bin=mb)
    ds.set_groups(counts)
    fit = ds.train(objective=3, use_quantized_grad=1, **kw)
    p, st = O.rank_params(counts, use_quantized_grad=1, **kw)
    ref = O.train(bins, n, 10, 64, y, p, missing_bin=mb)
    _compare_fit(fit, ref, n)


@pytest.mark.parametrize("quantized", [1, 0])
def test_training_lambdarank(dev, quantized):
    """A LambdaRank ensemble on the device against the oracle's restatement
    of train_ranker (ranking.mojo:690-771): quantized gradients bit-exact;
    fp32-path histograms (fp64 sums of the binary64 lambdas) within 1e-5."""
    x, y, counts, n = ranking_data(300)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, 10, max_bins=63)
    kw = dict(num_iterations=10, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    ds = dev.Dataset(bins, n, 10, 64, y, missing_bin=mb)
    ds.set_groups(counts)
    fit = ds.train(objective=3, use_quantized_grad=quantized, **kw)
    p, st = O.rank_params(counts, use_quantized_grad=quantized, **kw)
    ref = O.train(bins, n, 10, 64, y, p, missing_bin=mb)
    assert fit.base[0] == 0.0 and fit.n_trees == ref.n_trees
    if quantized:
        _compare_fit(fit, ref, n)
    else:
        assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
        assert _tree_agreement(fit, ref) >= ref.n_trees - 1


def test_ranker_estimator_through_c_abi(dev, tmp_path):
    """MojoTreesRanker(device="gpu").fit(X, y, group) -> mbh_train_ranker_dense:
    the model ranks better than chance, predicts the same bits on the host
    and the device, and survives save/load (objective 7)."""
    from mojoboost_amd.sklearn import MojoTreesRanker

    x, y, counts, n = ranking_data(200, seed=47)
    X = np.ascontiguousarray(x.T)
    est = MojoTreesRanker(n_estimators=20, num_leaves=15, learning_rate=0.2, max_bin=63,
                          min_child_samples=5).fit(X, y, group=counts)
    s_cpu = est.predict(X)
    s_gpu = est.predict(X, device="gpu")
    assert np.array_equal(bits(s_cpu), bits(s_gpu))
    # within every query the score order agrees with the grade more often than not
    agree, total, a = 0, 0, 0
    for c in counts:
        ss, yy = s_cpu[a:a + c], y[a:a + c]
        i, j = np.triu_indices(c, 1)
        m = yy[i] != yy[j]
        agree += int(np.sum(np.sign(ss[i] - ss[j])[m] == np.sign(yy[i] - yy[j])[m]))
        total += int(m.sum())
        a += c
    assert agree > 0.75 * total
    path = tmp_path / "ranker.txt"
    est.save(str(path))
    assert "objective 7" in path.read_text()
    back = MojoTreesRanker.load(str(path))
    assert np.array_equal(bits(back.predict(X)), bits(s_cpu))
