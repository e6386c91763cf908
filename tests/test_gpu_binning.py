"""The device binning transform (mbh_bin_dense_device, mb_binning.hip)
against the host binning (mbh_bin_dense / mbh_bin_dense_cat, pinned to the
oracle's fit_bins + transform by tests/test_binning_sampled.py), byte for
byte: the C2 shape at its full 10.5M x 28, and a small matrix built to hit
every arm of BinMapper.transform (src/mojotrees/binning.mojo:3242-3330) and
CategoricalSpec.bin_of (src/mojotrees/categorical.mojo:296-322) -- values
equal to an edge, +-inf, NaN with and without a reserved missing bin, a
constant column, a two-level column, and category codes that are negative,
fractional, unseen, NaN, -inf or 2^31 - 1."""
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


def test_c2_full_size_device_transform_equals_host(dev):
    import bench

    n, f = 10_500_000, 28
    x, _ = bench.c2_data(n)
    x = np.ascontiguousarray(x, np.float64)
    want, wmb = dev.bin_dense(x.ravel(), n, f, max_bins=255)
    got, gmb, gnc, t = dev.bin_dense_device(x.ravel(), n, f, max_bins=255)
    assert np.array_equal(gmb, wmb)
    assert not gnc.any()
    assert np.array_equal(got, want)
    assert t["transform_ms"] > 0.0


def _arms_matrix(n=50_000, seed=9):
    rng = np.random.default_rng(seed)
    cols = []
    a = rng.normal(size=n)
    a[rng.uniform(size=n) < 0.05] = np.nan              # NaN -> reserved missing bin
    cols.append(a)
    b = np.round(rng.normal(size=n), 1)                 # many values equal to an edge
    b[:7] = [np.inf, -np.inf, 0.0, -0.0, 1e308, -1e308, 5e-324]
    cols.append(b)
    cols.append(np.full(n, 3.25))                       # constant column
    c = np.where(rng.uniform(size=n) < 0.5, 1.0, 2.0)   # two levels
    cols.append(c)
    d = rng.integers(0, 40, size=n).astype(np.float64)  # categorical codes
    # (a code of 2^31 or more is refused by the fit, so only the transform of
    # other data could meet one)
    d[:10] = [-1.0, -0.5, 0.5, 39.9, 2.0 ** 31 - 1, np.nan, -np.inf, -1e300, 0.0, 7.0]
    cols.append(d)
    e = rng.exponential(size=n)
    cols.append(e)
    x = np.vstack(cols)
    return x, n, x.shape[0]


@pytest.mark.parametrize("use_missing", [True, False])
@pytest.mark.parametrize("max_bins", [255, 16, 2])
def test_every_transform_arm_equals_host(dev, use_missing, max_bins):
    x, n, f = _arms_matrix()
    cats = np.array([4], np.int32)
    want, wmb, wnc = dev.bin_dense(x.ravel(), n, f, max_bins=max_bins, use_missing=use_missing,
                                   sample_cnt=20_000, categorical=cats)
    got, gmb, gnc, _ = dev.bin_dense_device(x.ravel(), n, f, max_bins=max_bins, use_missing=use_missing,
                                            sample_cnt=20_000, categorical=cats)
    assert np.array_equal(gmb, wmb) and np.array_equal(gnc, wnc)
    assert np.array_equal(got, want)
    # NaN with no reserved bin is binned as 0.0 (the oracle's edges, which
    # equal the product's, give the bin of 0.0: the count of edges below it)
    if not use_missing:
        _, edges, k, omb = O.fit_transform(x[0].copy(), n, 1, max_bins=max_bins, use_missing=0,
                                           sample_cnt=20_000)
        assert omb[0] < 0 and wmb[0] < 0
        nan0 = np.isnan(x[0])
        assert nan0.any()
        assert np.all(got.reshape(f, n)[0][nan0] == int(np.sum(edges[0, :k[0]] < 0.0)))


def test_numeric_bins_equal_the_oracle_transform(dev):
    x, n, f = _arms_matrix(seed=10)
    x = x[[0, 1, 2, 3, 5]].copy()
    f = x.shape[0]
    want, _, _, wmb = O.fit_transform(x.ravel(), n, f, max_bins=255)
    got, gmb, _, _ = dev.bin_dense_device(x.ravel(), n, f, max_bins=255, sample_cnt=0)
    assert np.array_equal(gmb, wmb)
    assert np.array_equal(got, want)
