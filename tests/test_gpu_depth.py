"""Deeper GPU parity runs against the CPU oracle: the C2 shape at 1M rows over
100 trees (where the max-abs lattice is at its smallest), C5-shaped softmax
with category sets as the bench runs it, every lattice width and both
roundings, lambda_l1 > 0 on both gradient paths, the C3 shape at its full 28
features and 255 leaves, the empty-bag fallback of the quantizer, and a root
large enough for the root partition's own launch.
Quantized comparisons are bit for bit; fp32-gradient ones within 1e-5
relative."""
import numpy as np
import pytest

import oracle_lib as O
from test_gpu_categorical import compare as compare_cat
from test_gpu_magnitude import _splitmix64
from test_gpu_parity import _compare_fit, _rel_err, _tree_agreement, c2_like

pytestmark = pytest.mark.gpu
GOLDEN = 0x9E3779B97F4A7C15


@pytest.fixture(scope="module")
def dev():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return device


def test_c2_shape_1m_rows_100_trees_bit_exact(dev):
    n = 1_000_000
    bins, y, mb, nb = c2_like(n, seed=21)
    kw = dict(objective=1, num_iterations=100, num_leaves=255, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    fit = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    assert fit.n_trees == ref.n_trees == 100
    _compare_fit(fit, ref, n)


def test_root_partition_launch_of_large_tasks_bit_exact(dev):
    """A root over at least kPartChunkRoot x (2 x CUs) rows (8.4M on 256 CUs)
    is partitioned by its own launch of 16K-row tasks (the C2 shape takes it
    on every tree); trees, values and raw scores bit-exact to the oracle."""
    n = 8_700_000
    rng = np.random.default_rng(33)
    x = rng.normal(size=(4, n))
    y = (rng.uniform(size=n) < 1 / (1 + np.exp(-(x[0] * x[1] + 0.5 * x[2])))).astype(np.float64)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, 4, max_bins=63)
    del x
    kw = dict(objective=1, num_iterations=3, num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.1)
    fit = dev.Dataset(bins, n, 4, 63, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, 4, 63, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    assert fit.n_trees == ref.n_trees == 3
    _compare_fit(fit, ref, n)


def c5_bins(n, K=10, seed=5, n_cont=40, cards=(4, 7, 11, 16, 23, 31, 40, 48, 57, 64)):
    """C5-shaped data at a reduced row count: 40
    N(0,1) columns binned by fit_bins, 10 integer columns of cardinality 4-64
    binned as category tables (code c in bin 1 + c: every code is kept), 10
    classes by argmax of random linear scores plus per-category effects plus
    Gumbel noise."""
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n_cont, n))
    scores = 0.5 * rng.normal(size=(K, n_cont)) @ x
    codes = []
    for c in cards:
        v = rng.integers(0, c, size=n)
        codes.append(v)
        scores += 0.5 * rng.normal(size=(K, c))[:, v]
    y = np.argmax(scores + rng.gumbel(size=(K, n)), axis=0).astype(np.float64)
    cb, _, _, cmb = O.fit_transform(x.ravel(), n, n_cont, max_bins=255)
    bins = np.vstack([cb.reshape(n_cont, n)] + [(1 + v).astype(np.uint8)[None] for v in codes])
    mb = np.concatenate([cmb, np.full(len(cards), -1, np.int32)])
    ncat = np.array([0] * n_cont + list(cards), np.int32)
    return bins.ravel(), y, mb, ncat, n_cont + len(cards)


def test_softmax_with_category_sets_c5_shape_bit_exact(dev):
    n, K = 100_000, 10
    bins, y, mb, ncat, f = c5_bins(n, K)
    kw = dict(objective=2, num_class=K, num_iterations=3, num_leaves=63, min_data_in_leaf=20,
              lambda_l2=1.0, learning_rate=0.1)
    cat = dict(max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=10.0, cat_l2=10.0,
               min_data_per_group=100)
    ds = dev.Dataset(bins, n, f, 255, y, missing_bin=mb, n_categories=ncat)
    fit = ds.train(**kw, **cat)
    p = O.default_params(**kw, **cat, use_quantized_grad=1)
    p.n_categories = ncat.ctypes.data
    ref = O.train(bins, n, f, 255, y, p, missing_bin=mb)
    assert fit.n_trees == ref.n_trees == 3 * K
    assert fit.cat_bits.any(), "some node must split on a category set"
    compare_cat(fit, ref, n)


@pytest.mark.parametrize("B", [2, 16, 126])
@pytest.mark.parametrize("stochastic", [1, 0])
def test_lattice_widths_and_roundings_bit_exact(dev, B, stochastic):
    n = 100_000
    bins, y, mb, nb = c2_like(n, seed=B + stochastic)
    kw = dict(objective=1, num_iterations=6, num_leaves=63, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1, num_grad_quant_bins=B, stochastic_rounding=stochastic)
    fit = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


@pytest.mark.parametrize("l1", [0.5, 20.0])
def test_lambda_l1_quantized_bit_exact(dev, l1):
    n = 100_000
    bins, y, mb, nb = c2_like(n, seed=31)
    kw = dict(objective=1, num_iterations=6, num_leaves=63, min_data_in_leaf=20, lambda_l2=1.0,
              lambda_l1=l1, learning_rate=0.1)
    fit = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb).train(**kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    _compare_fit(fit, ref, n)


def test_lambda_l1_fp32(dev):
    n = 100_000
    bins, y, mb, nb = c2_like(n, f=16, seed=32)
    kw = dict(objective=1, num_iterations=20, num_leaves=63, min_data_in_leaf=20, lambda_l2=1.0,
              lambda_l1=2.0, learning_rate=0.1)
    fit = dev.Dataset(bins, n, 16, nb, y, missing_bin=mb).train(use_quantized_grad=0, **kw)
    ref = O.train(bins, n, 16, nb, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=mb)
    assert fit.n_trees == ref.n_trees
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(fit, ref) >= ref.n_trees - 1


def test_goss_fp32_c3_shape_full_width(dev):
    """C3's shape -- 28 features, 255 leaves, fp32 gradients, GOSS 0.2 / 0.1
    after floor(1 / 0.1) = 10 warmup rounds -- at 200k rows, 16 rounds."""
    n = 200_000
    bins, y, mb, nb = c2_like(n, seed=33)
    kw = dict(objective=1, num_iterations=16, num_leaves=255, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1)
    goss = dict(goss=1, top_rate=0.2, other_rate=0.1)
    fit = dev.Dataset(bins, n, 28, nb, y, missing_bin=mb).train(use_quantized_grad=0, **goss, **kw)
    ref = O.train(bins, n, 28, nb, y, O.default_params(**kw, **goss, use_quantized_grad=0), missing_bin=mb)
    assert fit.n_trees == ref.n_trees == 16
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(fit, ref) >= ref.n_trees - 1


def _bag(n, fraction, seed, bag_index):
    """bagging.sample_rows (src/mojotrees/bagging.mojo:101-129) with its
    empty-bag rule: no row drawn -> the row of the least draw."""
    import ctypes as C

    L = O.lib()
    L.orc_splitmix64.restype = C.c_uint64
    L.orc_splitmix64.argtypes = [C.c_uint64]
    stream = L.orc_splitmix64(((seed & 0x7FFFFFFFFFFFFFFF) ^ (bag_index * GOLDEN)) % 2 ** 64)
    with np.errstate(over="ignore"):
        ctr = np.uint64(stream) + np.arange(n, dtype=np.uint64)
    u = (_splitmix64(ctr) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    rows = np.flatnonzero(u < fraction)
    if len(rows) == 0:
        rows = np.array([int(np.argmin(u))])
    return rows.astype(np.int32), len(np.flatnonzero(u < fraction)) == 0


def test_quantizer_empty_bag_fallback_past_the_last_round(dev):
    """The device draws each round's bag; a bag with no row takes the row of
    the least draw (the host fills that table per bag). Rounds far past
    num_iterations must still read their own entry: the scales equal the
    oracle quantizer's over the oracle's bag, fallback included."""
    n, f = 300, 3
    rng = np.random.default_rng(8)
    bins = rng.integers(0, 8, size=(f, n), dtype=np.uint8)
    y = (rng.uniform(size=n) < 0.5).astype(np.float64)
    raw = rng.normal(size=n)
    ds = dev.Dataset(bins, n, f, 8, y)
    fraction, seed = 0.002, 4
    empties = 0
    for rnd in (0, 1, 7, 40, 123):
        g, h, qg, qh, sc = ds.objective_quantize(raw, round_index=rnd, objective=1, num_iterations=2,
                                                 bagging_fraction=fraction, bagging_freq=1,
                                                 bagging_seed=seed)
        og, oh = O.grad_hess(1, raw, y)
        rows, empty = _bag(n, fraction, seed, rnd)
        empties += empty
        oqg, oqh, osc = O.quantize(og, oh, rows=rows, quant_bins=4, stochastic=1, seed=11, round_index=rnd)
        assert sc[0] == osc[0] and sc[1] == osc[1], rnd
        assert np.array_equal(qg, oqg) and np.array_equal(qh, oqh)
    assert empties >= 2, "the case must exercise the empty-bag fallback"
