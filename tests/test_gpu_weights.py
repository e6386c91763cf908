"""GPU parity for sample weights (boosting._fill_grad_hess_into,
src/mojotrees/boosting.mojo:676-811; _base_score, :521-568): device training
with per-row weights against the CPU oracle with the same weights on the same
bins -- bit-exact on the quantized path for squared error, binary and
multiclass, the fp32 bar on the fp32 path -- and the estimators'
sample_weight through the C ABI.
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


def data(n, f, seed, objective, num_class=3):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(f, n))
    z = x[0] - 0.6 * x[1] * x[2] + 0.3 * x[3]
    if objective == 0:
        y = z + 0.1 * rng.normal(size=n)
    elif objective == 1:
        y = (rng.uniform(size=n) < 1 / (1 + np.exp(-z))).astype(float)
    else:
        y = np.digitize(z + 0.3 * rng.normal(size=n), [-0.5, 0.5]).astype(float)
    # weights in [0, 3), a tenth of them zero
    w = rng.uniform(0, 3, size=n)
    w[rng.uniform(size=n) < 0.1] = 0.0
    return x, y, w


@pytest.mark.parametrize("objective,leaves,trees", [(0, 63, 8), (1, 31, 8), (2, 15, 4)])
def test_weighted_training_bit_exact_quantized(dev, objective, leaves, trees):
    n, f = 150_000, 8
    x, y, w = data(n, f, 20 + objective, objective)
    bins, mb = dev.bin_dense(x.ravel(), n, f, max_bins=255)
    kw = dict(objective=objective, num_iterations=trees, num_leaves=leaves, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    if objective == 2:
        kw["num_class"] = 3
    fit = dev.Dataset(bins, n, f, 255, y, missing_bin=mb, weights=w).train(**kw)
    p, keep = O.weighted_params(w, **kw, use_quantized_grad=1)
    ref = O.train(bins, n, f, 255, y, p, missing_bin=mb)
    assert np.array_equal(bits(fit.base), bits(ref.base))
    assert fit.n_trees == ref.n_trees and np.array_equal(fit.off, ref.off)
    for k in ("feature", "threshold", "left", "right", "default_left", "missing_bin"):
        assert np.array_equal(getattr(fit, k), getattr(ref, k)), k
    for k in ("value", "gain", "count"):
        assert np.array_equal(bits(getattr(fit, k)), bits(getattr(ref, k))), k
    assert np.array_equal(bits(fit.train_raw()), bits(ref.train_raw(n)))


def test_weighted_training_fp32(dev):
    n, f = 80_000, 6
    x, y, w = data(n, f, 31, 1)
    bins, mb = dev.bin_dense(x.ravel(), n, f, max_bins=63)
    kw = dict(objective=1, num_iterations=6, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    fit = dev.Dataset(bins, n, f, 63, y, missing_bin=mb, weights=w).train(**kw, use_quantized_grad=0)
    p, keep = O.weighted_params(w, **kw, use_quantized_grad=0)
    ref = O.train(bins, n, f, 63, y, p, missing_bin=mb)
    assert np.array_equal(bits(fit.base), bits(ref.base))
    for k in ("feature", "threshold", "left", "right", "default_left"):
        assert np.array_equal(getattr(fit, k), getattr(ref, k)), k
    assert np.allclose(fit.value, ref.value, rtol=1e-5, atol=1e-12)
    assert np.allclose(fit.train_raw(), ref.train_raw(n), rtol=1e-5, atol=1e-9)


def test_weights_can_be_cleared(dev):
    n, f = 30_000, 5
    x, y, w = data(n, f, 41, 0)
    bins, mb = dev.bin_dense(x.ravel(), n, f, max_bins=63)
    ds = dev.Dataset(bins, n, f, 63, y, missing_bin=mb)
    kw = dict(objective=0, num_iterations=3, num_leaves=15)
    plain = ds.train(**kw)
    ds.set_weights(w)
    weighted = ds.train(**kw)
    ds.set_weights(None)
    again = ds.train(**kw)
    assert not np.array_equal(bits(plain.value), bits(weighted.value))
    assert np.array_equal(bits(plain.value), bits(again.value))


def test_estimators_sample_weight_through_c_abi(dev):
    from mojoboost_amd.sklearn import MojoTreesClassifier, MojoTreesRegressor

    n, f = 40_000, 6
    for objective, est in ((0, MojoTreesRegressor), (1, MojoTreesClassifier)):
        x, y, w = data(n, f, 50 + objective, objective)
        X = np.ascontiguousarray(x.T)
        m = est(n_estimators=6, num_leaves=31, max_bin=63, device="gpu", use_quantized_grad=True)
        m.fit(X, y, sample_weight=w)
        raw = m.predict(X, raw_score=True) if objective == 0 else m.decision_function(X)
        bins, mb = dev.bin_dense(x.ravel(), n, f, max_bins=63)
        p, keep = O.weighted_params(w, objective=objective, num_iterations=6, num_leaves=31,
                                    learning_rate=0.1, min_data_in_leaf=20, lambda_l2=1.0,
                                    min_sum_hessian=1e-3, use_quantized_grad=1)
        ref = O.train(bins, n, f, 63, y, p, missing_bin=mb)
        want, _ = ref.predict_binned(bins, n, f)
        assert np.array_equal(bits(raw), bits(want))


def ranking_data(n_queries, f=8, seed=61, max_q=120):
    rng = np.random.default_rng(seed)
    counts = rng.integers(1, max_q + 1, size=n_queries)
    n = int(counts.sum())
    x = rng.normal(size=(f, n))
    s = x[0] - 0.5 * x[1] + 0.3 * x[2] * x[3] + 0.5 * rng.normal(size=n)
    y = np.clip(np.floor((s + 2.0)), 0, 4).astype(np.float64)
    return x, y, counts.astype(np.int32), n


@pytest.mark.parametrize("n_queries,fraction,freq,weighted", [(300, 0.6, 2, True), (300, 0.5, 1, False),
                                                               (3, 0.05, 1, True)])
def test_lambdarank_query_bagging_and_weights_bit_exact(dev, n_queries, fraction, freq, weighted):
    """train_ranker with bagging and sample_weight (ranking.mojo:690-771):
    whole queries bagged, weights scaling the lambdas; quantized training
    bit-exact to the oracle. Three queries at fraction 0.05 draw empty bags,
    which take the query of the least draw (bagging.sample_rows)."""
    x, y, counts, n = ranking_data(n_queries)
    f = x.shape[0]
    bins, mb = dev.bin_dense(x.ravel(), n, f, max_bins=63)
    w = np.random.default_rng(5).uniform(0.2, 2.0, size=n) if weighted else None
    kw = dict(num_iterations=8, num_leaves=15, min_data_in_leaf=5, lambda_l2=1.0, learning_rate=0.1,
              bagging_fraction=fraction, bagging_freq=freq, bagging_seed=9)
    ds = dev.Dataset(bins, n, f, 63, y, missing_bin=mb, weights=w)
    ds.set_groups(counts)
    fit = ds.train(objective=3, use_quantized_grad=1, **kw)
    p, st = O.rank_params(counts, use_quantized_grad=1, **kw)
    if weighted:
        wk = np.ascontiguousarray(w)
        p.weights = wk.ctypes.data
    ref = O.train(bins, n, f, 63, y, p, missing_bin=mb)
    assert fit.n_trees == ref.n_trees > 0
    for k in ("feature", "threshold", "left", "right", "default_left"):
        assert np.array_equal(getattr(fit, k), getattr(ref, k)), k
    for k in ("value", "gain", "count"):
        assert np.array_equal(bits(getattr(fit, k)), bits(getattr(ref, k))), k
    assert np.array_equal(bits(fit.train_raw()), bits(ref.train_raw(n)))
