"""Sampled quantile binning (bin_construct_sample_rows + fit_bins,
src/mojotrees/binning.mojo:1745-1785, :3565-4047), pinned without the
reference, and the product's host binning against the oracle's.

What pins the oracle:
- the sample: exactly sample_cnt rows, strictly ascending, in range; none
  (every row) for sample_cnt <= 0 or >= n_rows; the selection's tail rule
  (the last rows are all taken once as many are needed as remain); each
  row's inclusion frequency over many seeds near sample_cnt / n_rows;
- the fit: the reference states that a sampled fit differs from a full one
  only in which values it reads -- the same ascending rows for every
  feature, missingness decided from what was read (binning.mojo:3796-3815).
  So fit_bins(x, sample_cnt) must equal the unsampled fit_bins of the
  sampled rows alone, edges, edge counts and missing bins, on a 1M-row
  matrix with NaNs, duplicate-heavy columns and rare levels; the golden
  `large` fixture pins the unsampled fit bit for bit
  (tests/test_oracle_golden.py).

The product (mbh_bin_dense, C++ in mb_host.cpp) must then produce the same
bins and missing bins as the oracle on the golden `large` input and on the
1M-row input (sampled), and mbh_bin_dense_cat the category bins of the
golden `misscat` input.
"""
import ctypes as C

import numpy as np
import pytest

import golden_fixtures as G
import oracle_lib as O
from mojoboost_amd import device


def _sample_rows(n, cnt, seed):
    L = O.lib()
    L.orc_bin_sample_rows.restype = C.c_int64
    L.orc_bin_sample_rows.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_void_p]
    out = np.zeros(max(1, min(n, max(cnt, 0))), np.int64)
    k = L.orc_bin_sample_rows(n, cnt, seed, out.ctypes.data_as(C.c_void_p))
    return out[:k]


@pytest.mark.parametrize("n,cnt", [(1000, 1), (1000, 10), (1000, 500), (1000, 998), (1000, 999),
                                   (250_000, 200_000), (1_000_003, 200_000)])
def test_sample_is_exact_and_ascending(n, cnt):
    rows = _sample_rows(n, cnt, seed=1)
    assert len(rows) == cnt
    assert rows[0] >= 0 and rows[-1] < n
    assert np.all(np.diff(rows) > 0)


@pytest.mark.parametrize("cnt", [0, -5, 1000, 5000])
def test_no_sample_means_every_row(cnt):
    assert len(_sample_rows(1000, cnt, seed=1)) == 0


def test_sample_tail_takes_every_remaining_row():
    """With need >= left the remaining rows are all taken: a sample of n - 1
    rows out of n skips exactly one row, and every row after the skipped one
    is present."""
    n = 50
    for seed in range(20):
        rows = _sample_rows(n, n - 1, seed)
        missing = sorted(set(range(n)) - set(rows.tolist()))
        assert len(missing) == 1
        assert rows.tolist() == [r for r in range(n) if r != missing[0]]


def test_sample_inclusion_is_uniform():
    n, cnt, seeds = 200, 50, 2000
    hits = np.zeros(n)
    for seed in range(seeds):
        hits[_sample_rows(n, cnt, seed)] += 1
    p = cnt / n
    sd = np.sqrt(seeds * p * (1 - p))
    assert np.all(np.abs(hits - seeds * p) < 5 * sd)
    assert np.abs(hits[:n // 2].sum() - hits[n // 2:].sum()) < 5 * np.sqrt(seeds * cnt)


def _big_matrix(n, seed=77):
    rng = np.random.default_rng(seed)
    f = 6
    x = np.empty((f, n))
    x[0] = rng.normal(size=n)
    x[1] = rng.normal(size=n)
    x[1, rng.uniform(size=n) < 0.03] = np.nan          # missing values
    x[2] = np.round(rng.normal(size=n), 1)             # duplicate-heavy
    x[3] = rng.integers(0, 20, size=n)                 # few levels
    rare = rng.uniform(size=n) < 0.0004
    x[3, rare] = 100 + rng.integers(0, 40, size=rare.sum())   # rare levels
    x[4] = rng.exponential(size=n)
    x[5] = rng.normal(size=n)
    x[5, :50] = np.nan                                  # NaN in a few early rows only
    return x, f


@pytest.fixture(scope="module")
def big():
    n = 1_000_000
    x, f = _big_matrix(n)
    return x, n, f


def test_sampled_fit_equals_the_fit_of_the_sampled_rows(big):
    x, n, f = big
    cnt, seed = 200_000, 3
    rows = _sample_rows(n, cnt, seed)
    sub = np.ascontiguousarray(x[:, rows])
    _, e1, k1, m1 = O.fit_transform(x.ravel(), n, f, max_bins=255, sample_cnt=cnt, seed=seed)
    _, e2, k2, m2 = O.fit_transform(sub.ravel(), cnt, f, max_bins=255, sample_cnt=0, seed=seed)
    assert np.array_equal(k1, k2)
    assert np.array_equal(m1, m2)
    for j in range(f):
        assert np.array_equal(e1[j, :k1[j]].view(np.uint64), e2[j, :k2[j]].view(np.uint64))
    # the sample decides missingness: column 5's NaNs sit in rows 0..49
    in_sample = np.isin(np.arange(50), rows).any()
    assert (m1[5] >= 0) == bool(in_sample)
    # and a different seed reads other rows and fits other edges
    _, e3, k3, _ = O.fit_transform(x.ravel(), n, f, max_bins=255, sample_cnt=cnt, seed=seed + 1)
    assert not np.array_equal(e1[0, :k1[0]], e3[0, :k3[0]])


def test_product_binning_equals_oracle_sampled(big):
    x, n, f = big
    want, _, _, wmb = O.fit_transform(x.ravel(), n, f, max_bins=255, sample_cnt=200_000, seed=1)
    got, gmb = device.bin_dense(x.ravel(), n, f, max_bins=255, sample_cnt=200_000, seed=1)
    assert np.array_equal(gmb, wmb)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("max_bins", [255, 63, 16])
def test_product_binning_equals_oracle_on_the_golden_large_input(max_bins):
    x, n, f, _, _, _ = G.fixture("large")
    want, _, _, wmb = O.fit_transform(x, n, f, max_bins=max_bins)
    got, gmb = device.bin_dense(x, n, f, max_bins=max_bins)
    assert np.array_equal(gmb, wmb)
    assert np.array_equal(got, want)


def test_product_category_bins_on_the_golden_misscat_input():
    x, n, f, _, (_, nb, cats), _ = G.fixture("misscat")
    got, gmb, ncat = device.bin_dense(x, n, f, max_bins=nb, categorical=cats)
    want, _, _, wmb = O.fit_transform(x, n, f, max_bins=nb)
    got = got.reshape(f, n)
    want = want.reshape(f, n)
    codes = x[2 * n:3 * n]
    assert list(ncat) == [0, 0, 6, 0, 0]
    assert np.array_equal(got[2], 1 + codes.astype(np.int64))   # code c -> bin 1 + rank
    assert gmb[2] == -1
    for j in (0, 1, 3, 4):
        assert np.array_equal(got[j], want[j])
        assert gmb[j] == wmb[j]
    assert gmb[1] >= 0          # feature 1 holds NaNs: a missing bin is reserved


@pytest.mark.parametrize("n_features", [1, 6])
def test_refused_categorical_code_is_an_error_not_an_abort(n_features):
    """The fit refuses a category code of 2^31 or more (the reference's
    categorical table is int32). The refusal is thrown on one of the host's
    fitting threads and must come back as the entry point's error."""
    n = 5000
    x = np.zeros((n_features, n))
    x[-1] = np.arange(n) % 7
    x[-1, 123] = 2.0 ** 31
    with pytest.raises(Exception, match="below 2\\^31"):
        device.bin_dense(x.ravel(), n, n_features, max_bins=16,
                         categorical=np.array([n_features - 1], np.int32))
