"""Parity at BASELINE.json's full sizes.

C2 (the north star's target): 10.5M x 28 binary logistic, 255 bins, 255
leaves, int8 quantized gradients, all 500 trees bit-identical to the CPU
oracle -- node for node, value, gain and count bits -- and the final raw
scores too. C4 at its full 400k x 2000 (12 trees) and C5 at its full 2M x 50
with category sets (8 rounds, 80 trees), likewise bit for bit. The oracle's
fits of these were made once on the CPU (tests/golden/make_full_size_digests.py)
and are compared as per-tree digests (tests/golden/full_size_digests.json);
the data are the bench's seeded generators, binned by the library's host
binning, and the test checks the bins' digest first so a data difference is
told apart from a training one.

C3 (fp32 gradients, GOSS 0.2 / 0.1 from round 10) at 1M rows x 100 trees
runs the oracle here: predictions after 100 trees within 1e-5 relative
and at least 99 of the 100 trees identical in
structure (fp64 sums in another order may move a near-tie split).
"""
import numpy as np
import pytest

import full_size as FS
import oracle_lib as O
from bench import c2_data
from test_gpu_parity import _rel_err, _tree_agreement

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return device


def _check_full(dev, name):
    want = FS.load()[name]
    bins, missing, ncat, y, n, F, nb = FS.data(name)
    print(f"[full-size] {name}: {n} x {F} binned, training {want['n_trees']} trees", flush=True)
    assert FS.sha(bins, np.asarray(missing, np.int32)) == want["bins_sha256"], "binned data differ"
    assert FS.sha(np.asarray(y, np.float64)) == want["labels_sha256"], "labels differ"
    ds = dev.Dataset(bins, n, F, nb, y, missing_bin=missing, n_categories=ncat)
    del bins
    fit = ds.train(num_grad_quant_bins=4, stochastic_rounding=1, **want["params"])
    assert fit.n_trees == want["n_trees"]
    assert [f"{int(v):016x}" for v in np.asarray(fit.base, np.float64).view(np.uint64)] == want["base_bits"]
    got = FS.tree_digests(fit)
    bad = [t for t, (a, b) in enumerate(zip(got, want["trees"])) if a != b]
    assert not bad, f"{len(bad)} of {fit.n_trees} trees differ from the oracle, the first is tree {bad[0]}"
    assert FS.sha(fit.train_raw().view(np.uint64)) == want["train_raw_sha256"], "final raw scores differ"
    ds.free()


def test_c2_full_size_500_trees_bit_exact(dev):
    _check_full(dev, "c2")


def test_c4_full_size_bit_exact(dev):
    _check_full(dev, "c4")


def test_c5_full_size_category_sets_bit_exact(dev):
    _check_full(dev, "c5")


def test_c3_goss_fp32_1m_rows_100_trees(dev):
    n = 1_000_000
    x, y = c2_data(n)
    bins, missing = dev.bin_dense(x.ravel(), n, 28, max_bins=255)
    del x
    kw = dict(objective=1, num_iterations=100, num_leaves=255, min_data_in_leaf=20, lambda_l2=1.0,
              learning_rate=0.1, goss=1, top_rate=0.2, other_rate=0.1)
    fit = dev.Dataset(bins, n, 28, 255, y, missing_bin=missing).train(use_quantized_grad=0, **kw)
    ref = O.train(bins, n, 28, 255, y, O.default_params(**kw, use_quantized_grad=0), missing_bin=missing)
    assert fit.n_trees == ref.n_trees == 100
    assert _rel_err(fit.train_raw(), ref.train_raw(n)) < 1e-5
    assert _tree_agreement(fit, ref) >= 99
