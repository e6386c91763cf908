"""Both leaf-row representations of the grower against the CPU oracle, bit
for bit: leaves holding their rows as records (partition_mode=1: the
partition moves each row's whole record, with its int8 pair, into the
child's contiguous range, and the histogram streams the records) and as row
ids (partition_mode=2: the partition moves 4-byte ids, the histogram gathers
records by id). Covered for records of 16, 32 and 64 bytes, unsampled roots
(row id = position), sampled roots (bagging, GOSS: the root list), missing
values, category sets and multiclass; a layout that cannot move records
(fp32 gradients) trains on row ids whatever the mode asks.
"""
import numpy as np
import pytest

import oracle_lib as O
from test_gpu_categorical import compare as compare_cat
from test_gpu_depth import c5_bins
from test_gpu_parity import _compare_fit, _rel_err, _tree_agreement, c2_like

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return device


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("f,leaves,extra", [
    (28, 255, {}),                                                  # 32-byte records, C2's shape
    (8, 31, dict(bagging_fraction=0.6, bagging_freq=1, bagging_seed=5)),  # 16-byte records, bagged roots
    (40, 63, {}),                                                   # 64-byte records
    (16, 63, dict(goss=1, top_rate=0.2, other_rate=0.1)),          # GOSS sample as the root list
])
def test_partition_modes_bit_exact(dev, mode, f, leaves, extra):
    n = 150_000
    lr = 0.25 if extra.get("goss") else 0.1
    bins, y, mb, nb = c2_like(n, f=min(f, 28), seed=70 + f)
    if f > 28:  # widen with shifted copies of the columns (more features per record)
        bins = np.concatenate([bins, np.roll(bins.reshape(28, n)[: f - 28], 17, axis=1).ravel()])
        mb = np.concatenate([mb, mb[: f - 28]])
    kw = dict(objective=1, num_iterations=8, num_leaves=leaves, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=lr, **extra)
    fit = dev.Dataset(bins, n, f, nb, y, missing_bin=mb).train(partition_mode=mode, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_record_partition_with_missing_values_and_tiny_leaves(dev):
    """NaN-binned rows route by default_left; min_data_in_leaf=1 lets leaves
    of one row move and accumulate."""
    n, f = 20_000, 6
    rng = np.random.default_rng(91)
    x = rng.normal(size=(f, n))
    x[rng.uniform(size=(f, n)) < 0.15] = np.nan
    y = (np.nan_to_num(x[0]) + np.nan_to_num(x[1]) * np.nan_to_num(x[2]) > 0.2).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=63)
    kw = dict(objective=1, num_iterations=6, num_leaves=127, min_data_in_leaf=1, lambda_l2=1.0,
              learning_rate=0.2)
    fit = dev.Dataset(bins, n, f, 63, y, missing_bin=mb).train(partition_mode=1, **kw)
    ref = O.train(bins, n, f, 63, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_record_partition_softmax_with_category_sets(dev):
    """C5's shape (50 features: 64-byte records, 10 category-set columns,
    10 classes) with records forced on: every class tree bit-exact."""
    n, K = 100_000, 10
    bins, y, mb, ncat, f = c5_bins(n, K, seed=17)
    kw = dict(objective=2, num_class=K, num_iterations=2, num_leaves=63, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    ds = dev.Dataset(bins, n, f, 255, y, missing_bin=mb, n_categories=ncat)
    fit = ds.train(partition_mode=1, **kw)
    p = O.default_params(**kw, use_quantized_grad=1)
    p.n_categories = ncat.ctypes.data
    ref = O.train(bins, n, f, 255, y, p, missing_bin=mb)
    compare_cat(fit, ref, n)


def test_fp32_path_ignores_the_record_mode(dev):
    """fp32 gradients keep row ids (their derivatives are gathered by id);
    asking for records changes nothing."""
    n, f = 60_000, 12
    bins, y, mb, nb = c2_like(n, f=f, seed=3)
    kw = dict(objective=1, num_iterations=6, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    ds = dev.Dataset(bins, n, f, nb, y, missing_bin=mb)
    a = ds.train(use_quantized_grad=0, partition_mode=1, **kw)
    ref = O.train(bins, n, f, nb, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=mb)
    assert _rel_err(a.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(a, ref) >= ref.n_trees - 1
