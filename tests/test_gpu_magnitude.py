"""GPU parity of the magnitude-sum power-of-two lattice (quant_scale_rule=1):
the reference's device magnitude reduction and scale
(gpu_objectives_native._abs_sum_kernel + sum_abs_partials :982-1125,
quantized_gradient.fixed_point_scale_pow2 :908-1117) and its 2^30-lattice
quantizer into int32 pairs (gpu_active_rows._quantize_grad_hess_kernel
:2211-2255), through int32 histograms to whole trees, against the CPU oracle.
Every comparison is on integers or IEEE-754 bit patterns.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from test_gpu_parity import _compare_fit, bits, c2_like

pytestmark = pytest.mark.gpu

GOLDEN = 0x9E3779B97F4A7C15


@pytest.fixture(scope="module")
def dev():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return device


def _splitmix64(x):
    x = np.asarray(x, np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _bag_mask(n, fraction, seed, bag_index):
    """bagging.sample_rows (src/mojotrees/bagging.mojo:101-129): row r is in
    the bag when uniform(stream + r) < fraction; the stream comes from the
    oracle's splitmix64 and the per-row draws are checked against its
    uniform."""
    L = O.lib()
    L.orc_splitmix64.restype = C.c_uint64
    L.orc_splitmix64.argtypes = [C.c_uint64]
    L.orc_uniform.restype = C.c_double
    L.orc_uniform.argtypes = [C.c_uint64]
    stream = L.orc_splitmix64(((seed & 0x7FFFFFFFFFFFFFFF) ^ (bag_index * GOLDEN)) % 2 ** 64)
    with np.errstate(over="ignore"):
        ctr = np.uint64(stream) + np.arange(n, dtype=np.uint64)
    u = (_splitmix64(ctr) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    for r in (0, 1, n // 2, n - 1):
        assert u[r] == L.orc_uniform((stream + r) % 2 ** 64)
    m = (u < fraction).astype(np.uint8)
    assert m.any()
    return m


@pytest.mark.parametrize("objective,stochastic,bagged",
                         [(0, 1, False), (1, 1, False), (1, 0, False), (1, 1, True), (0, 0, True)])
def test_magnitude_sums_scales_and_quantizer_bit_exact(dev, objective, stochastic, bagged):
    n, f = 300_007, 4   # more rows than the reduction's 65536 threads, several times
    rng = np.random.default_rng(40 + objective)
    bins = rng.integers(0, 16, size=(f, n), dtype=np.uint8)
    y = (rng.uniform(size=n) < 0.4).astype(np.float64) if objective == 1 else rng.normal(size=n)
    raw = rng.normal(0, 2, size=n)
    ds = dev.Dataset(bins, n, f, 16, y)
    kw = dict(objective=objective, quant_scale_rule=1, stochastic_rounding=stochastic)
    if bagged:
        kw.update(bagging_fraction=0.6, bagging_freq=1, bagging_seed=5)
    for rnd in (0, 3):
        g, h, qg, qh, sc = ds.objective_quantize32(raw, round_index=rnd, **kw)
        og, oh = O.grad_hess(objective, raw, y)
        assert np.array_equal(g.astype(np.float64), og)
        assert np.array_equal(h.astype(np.float64), oh)
        mask = _bag_mask(n, 0.6, 5, rnd) if bagged else None
        sg, sh = O.magnitude_sums(og, oh, mask)
        assert sc[2] == sg and sc[3] == sh
        rows = None if mask is None else np.flatnonzero(mask).astype(np.int32)
        oqg, oqh, osc = O.quantize_rule(og, oh, O.RULE_MAGNITUDE_SUM, rows=rows, stochastic=stochastic,
                                        seed=11, round_index=rnd,
                                        const_hessian=1 if objective == 0 else 0)
        assert sc[0] == osc[0] and sc[1] == osc[1]
        assert sc[0] == O.fixed_point_scale_pow2(sg)
        assert np.array_equal(qg, oqg)
        assert np.array_equal(qh, oqh)


@pytest.mark.parametrize("subset", [False, True])
def test_int32_histogram_bit_exact(dev, subset):
    n, f, nb = 300_000, 28, 255
    rng = np.random.default_rng(17)
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    bins[5] %= 3                                   # hot bins
    qg = rng.integers(-3000, 3001, size=n).astype(np.int32)
    qh = rng.integers(0, 3001, size=n).astype(np.int32)
    qg[:10] = [2 ** 20, -2 ** 20, 2 ** 19, 7, -7, 0, 1, -1, 2 ** 21, -2 ** 21]
    ds = dev.Dataset(bins, n, f, nb, np.zeros(n))
    rows = np.sort(rng.choice(n, 123_457, replace=False)).astype(np.int32) if subset else None
    got = ds.histogram32(qg, qh, rows)
    want = O.hist_quantized32(bins.ravel(), n, f, nb, qg, qh, rows)
    assert np.array_equal(got.astype(np.int64), want)


def _train_both(dev, bins, n, f, nb, y, mb, **kw):
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    fit = ds.train(quant_scale_rule=1, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1, quant_scale_rule=1),
                  missing_bin=mb)
    return fit, ref


def test_training_c2_shape_magnitude_lattice_bit_exact(dev):
    n = 200_000
    bins, y, mb, nb = c2_like(n, seed=3)
    fit, ref = _train_both(dev, bins, n, 28, nb, y, mb, objective=1, num_iterations=10, num_leaves=255,
                           min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.1)
    _compare_fit(fit, ref, n)


def test_training_regression_nearest_rounding_magnitude_lattice(dev):
    """Squared error (a constant hessian: one unit over max|h|) with
    round-to-nearest, the rounding the reference's device quantizer uses."""
    n, f, nb = 80_000, 10, 63
    rng = np.random.default_rng(23)
    x = rng.normal(size=(f, n))
    y = x[0] - 2 * x[1] * x[2] + 0.1 * rng.normal(size=n)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=nb)
    fit, ref = _train_both(dev, bins, n, f, nb, y, mb, objective=0, num_iterations=8, num_leaves=31,
                           min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.1, stochastic_rounding=0)
    _compare_fit(fit, ref, n)


def test_training_multiclass_bagged_magnitude_lattice(dev):
    """One lattice per class (derive_multiclass_scales), each from its own
    class's sampled magnitudes."""
    n, f, nb = 60_000, 8, 63
    rng = np.random.default_rng(29)
    x = rng.normal(size=(f, n))
    y = np.argmax(np.stack([x[0], x[1] - x[2], 0.5 * x[3]]) + rng.gumbel(size=(3, n)), axis=0).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=nb)
    fit, ref = _train_both(dev, bins, n, f, nb, y, mb, objective=2, num_class=3, num_iterations=4,
                           num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.2,
                           bagging_fraction=0.7, bagging_freq=1, bagging_seed=6, feature_fraction=0.8)
    _compare_fit(fit, ref, n)


def test_magnitude_lattice_through_the_c_abi(dev):
    """The parameter string's quant_scale_rule=magnitude_sum reaches the
    device lattice: the estimator's raw scores equal the oracle's."""
    from mojoboost_amd.sklearn import MojoTreesRegressor

    n, f = 40_000, 6
    rng = np.random.default_rng(31)
    X = rng.normal(size=(n, f))
    y = X[:, 0] * X[:, 1] + 0.1 * rng.normal(size=n)

    class Est(MojoTreesRegressor):
        def _params(self, extra=""):
            return super()._params(extra) + " quant_scale_rule=magnitude_sum"

    est = Est(n_estimators=5, num_leaves=15, max_bin=63, device="gpu", use_quantized_grad=True).fit(X, y)
    raw = est.predict(X)
    x_cm = np.ascontiguousarray(X.T).ravel()
    bins, _, _, mb = O.fit_transform(x_cm, n, f, max_bins=63)
    p = O.default_params(objective=0, num_iterations=5, num_leaves=15, learning_rate=0.1, min_data_in_leaf=20,
                         lambda_l2=1.0, min_sum_hessian=1e-3, use_quantized_grad=1, stochastic_rounding=1,
                         quant_scale_rule=1)
    ref = O.train(bins, n, f, 64, y, p, missing_bin=mb)
    want, _ = ref.predict_binned(bins, n, f)
    assert np.array_equal(bits(raw), bits(want))


@pytest.mark.parametrize("n", [300_000, 6_000])
def test_int16_staging_values_and_misfit_counts(dev, n):
    """The packed int16 arm (_quantize_grad_hess_i16_kernel,
    gpu_active_rows.mojo:2298-2352): the staged values are the int32
    lattice's integers narrowed to 16 bits, and the per-plane counters count
    exactly the values outside [-32768, 32767]. At 300k logistic rows every
    value fits (max|g| / sum|g| is near 1 / n); at 6k rows many do not."""
    f = 4
    rng = np.random.default_rng(n)
    bins = rng.integers(0, 16, size=(f, n), dtype=np.uint8)
    y = (rng.uniform(size=n) < 0.4).astype(np.float64)
    raw = rng.normal(0, 2, size=n)
    ds = dev.Dataset(bins, n, f, 16, y)
    g, h, qg, qh, sc = ds.objective_quantize32(raw, objective=1, quant_scale_rule=1, quant_staging=1)
    og, oh = O.grad_hess(1, raw, y)
    oqg, oqh, _ = O.quantize_rule(og, oh, O.RULE_MAGNITUDE_SUM, stochastic=1, seed=11)
    misfit_g = int(np.sum((oqg > 32767) | (oqg < -32768)))
    misfit_h = int(np.sum((oqh > 32767) | (oqh < -32768)))
    assert (sc[4], sc[5]) == (misfit_g, misfit_h)
    assert np.array_equal(qg, oqg.astype(np.int16).astype(np.int32))
    assert np.array_equal(qh, oqh.astype(np.int16).astype(np.int32))
    if n == 300_000:
        assert misfit_g == misfit_h == 0
    else:
        assert misfit_g > 0


def test_training_int16_staging_equals_int32_staging(dev):
    n = 300_000
    bins, y, mb, nb = c2_like(n, seed=9)
    kw = dict(objective=1, num_iterations=8, num_leaves=255, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1, quant_scale_rule=1)
    ds = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb)
    a = ds.train(quant_staging=1, **kw)
    b = ds.train(quant_staging=0, **kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**{k: v for k, v in kw.items()},
                                                       use_quantized_grad=1), missing_bin=mb)
    _compare_fit(a, ref, n)
    _compare_fit(b, ref, n)


def test_int16_staging_refuses_a_misfit(dev):
    from mojoboost_amd._lib import ERROR_TRAINING, MojoTreesError

    n, f = 3_000, 4
    rng = np.random.default_rng(2)
    bins = rng.integers(0, 16, size=(f, n), dtype=np.uint8)
    y = (rng.uniform(size=n) < 0.5).astype(np.float64)
    ds = dev.Dataset(bins, n, f, 16, y)
    with pytest.raises(MojoTreesError) as e:
        ds.train(objective=1, num_iterations=2, num_leaves=7, quant_scale_rule=1, quant_staging=1)
    assert e.value.code == ERROR_TRAINING and "int16" in e.value.message
    # the same fit on the int32 staging trains
    assert ds.train(objective=1, num_iterations=2, num_leaves=7, quant_scale_rule=1).n_trees == 2
