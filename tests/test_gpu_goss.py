"""GOSS on the quantized path and with multiclass, against the CPU oracle.

The reference samples first and quantizes second: goss_round
(src/mojotrees/goss.mojo:376-396) weights the sampled small-gradient rows'
derivatives in binary64, and the grower's quantizer then sees the weighted
derivatives of the sampled rows only. A multiclass round draws one sample
from the class sum of |g_k h_k| (boosting._multiclass_goss_select,
boosting.mojo:3680-3710) and grows every class's tree on it (:4041-4053).
Quantized fits are compared bit for bit; fp32 ones within 1e-5 relative
with the trees' structure."""
import numpy as np
import pytest

import oracle_lib as O
from test_gpu_parity import _compare_fit, _rel_err, _tree_agreement, c2_like, c5_like

pytestmark = pytest.mark.gpu
GOSS = dict(goss=1, top_rate=0.2, other_rate=0.1)


@pytest.fixture(scope="module")
def dev():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return device


@pytest.mark.parametrize("objective,n,f,leaves,lr,iters", [
    (1, 3_000, 4, 15, 0.25, 12),     # small: the sampling's one-by-one steps are frequent
    (1, 200_000, 16, 63, 0.25, 10),
    (0, 100_000, 8, 31, 0.5, 8),     # L2: GOSS weights the hessians (no constant hessian)
])
def test_quantized_goss_bit_exact(dev, objective, n, f, leaves, lr, iters):
    bins, y, mb, nb = c2_like(n, f=f, seed=40 + f)
    if objective == 0:
        y = y * 2.0 - 0.5 + 0.1 * np.random.default_rng(1).normal(size=n)
    kw = dict(objective=objective, num_iterations=iters, num_leaves=leaves, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=lr)
    fit = dev.Dataset(bins, n, f, nb, y, missing_bin=mb).train(**GOSS, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, **GOSS, use_quantized_grad=1), missing_bin=mb)
    warm = int(1.0 / lr)
    assert ref.n_trees == iters and iters > warm
    # rounds past the warmup grew on the sample
    assert ref.tree(warm)["count"][0] < n
    _compare_fit(fit, ref, n)


def test_quantized_goss_c3_shape(dev):
    """C3's shape -- 28 features, 255 leaves, GOSS 0.2 / 0.1 after
    floor(1 / 0.1) = 10 warmup rounds -- quantized, at 200k rows, 14 rounds."""
    n = 200_000
    bins, y, mb, nb = c2_like(n, seed=45)
    kw = dict(objective=1, num_iterations=14, num_leaves=255, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    fit = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb).train(**GOSS, **kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**kw, **GOSS, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


@pytest.mark.parametrize("quantized", [1, 0])
def test_multiclass_goss(dev, quantized):
    n, K = 100_000, 4
    bins, y, mb, nb, f = c5_like(n, K, seed=46)
    kw = dict(objective=2, num_class=K, num_iterations=6, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.5)
    fit = dev.Dataset(bins, n, f, nb, y, missing_bin=mb).train(use_quantized_grad=quantized, **GOSS, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, **GOSS, use_quantized_grad=quantized),
                  missing_bin=mb)
    assert ref.n_trees == fit.n_trees == 6 * K
    roots = np.array([ref.tree(t)["count"][0] for t in range(ref.n_trees)]).reshape(-1, K)
    assert np.all(roots[2:] < n) and np.all(roots[2:] == roots[2:, :1])  # one sample per round
    if quantized:
        _compare_fit(fit, ref, n)
    else:
        assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
        assert _tree_agreement(fit, ref) >= ref.n_trees - 1


@pytest.mark.parametrize("objective,staging", [(1, 0), (0, 0), (1, 1)])
def test_goss_on_the_magnitude_sum_lattice(dev, objective, staging):
    """GOSS with the reference's magnitude-sum lattice (quant_scale_rule=1,
    the 2^30 power-of-two scales): the magnitude sums cover the round's
    sample with the GOSS weight applied to the kept small-gradient rows, the
    quantizer sees the weighted derivatives; int32 and int16 staging.
    Every tree and raw score bit-exact to the oracle. The int16 arm needs
    rows enough for every weighted row's value to fit 16 bits at the
    sample's scale (it refuses the fit otherwise): 1.5M rows there."""
    n = 1_500_000 if staging else 60_000
    bins, y, mb, nb = c2_like(n, f=8, seed=48 + objective)
    if objective == 0:
        y = y * 2.0 - 0.5 + 0.1 * np.random.default_rng(2).normal(size=n)
    kw = dict(objective=objective, num_iterations=8, num_leaves=31, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.25)
    fit = dev.Dataset(bins, n, 8, nb, y, missing_bin=mb).train(quant_scale_rule=1, quant_staging=staging,
                                                               **GOSS, **kw)
    ref = O.train(bins, n, 8, nb, y, O.default_params(**kw, **GOSS, use_quantized_grad=1, quant_scale_rule=1),
                  missing_bin=mb)
    assert ref.n_trees == 8 and ref.tree(5)["count"][0] < n  # rounds past the warmup sampled
    _compare_fit(fit, ref, n)


def test_multiclass_goss_on_the_magnitude_sum_lattice(dev):
    n, K = 60_000, 3
    bins, y, mb, nb, f = c5_like(n, K, seed=49)
    kw = dict(objective=2, num_class=K, num_iterations=5, num_leaves=15, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.5)
    fit = dev.Dataset(bins, n, f, nb, y, missing_bin=mb).train(quant_scale_rule=1, **GOSS, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, **GOSS, use_quantized_grad=1, quant_scale_rule=1),
                  missing_bin=mb)
    assert ref.n_trees == fit.n_trees == 5 * K
    _compare_fit(fit, ref, n)
