"""Quantized-gradient path of the oracle: the integer histogram, the
integer split search and quantized training.

The reference never connects its quantizer to a trainer
(src/mojotrees/quantized_gradient.mojo:256, CONNECTED = False), so no
reference vector exists for these; they are pinned by brute force
(numpy scatter-add, exhaustive candidate enumeration) and invariants.
"""
import itertools

import numpy as np
import pytest

import oracle_lib as O


def _data(n, f, nb, seed):
    rng = np.random.default_rng(seed)
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    qg = rng.integers(-2, 3, size=n).astype(np.int8)
    qh = rng.integers(0, 5, size=n).astype(np.int8)
    return bins, qg, qh


def test_integer_histogram_matches_scatter_add():
    n, f, nb = 5000, 7, 33
    bins, qg, qh = _data(n, f, nb, 1)
    rows = np.sort(np.random.default_rng(2).choice(n, 1234, replace=False)).astype(np.int32)
    for sel in (None, rows):
        h = O.hist_quantized(bins.ravel(), n, f, nb, qg, qh, sel)
        idx = np.arange(n) if sel is None else sel
        for ff in range(f):
            want = np.zeros((nb, 3), np.int64)
            np.add.at(want[:, 0], bins[ff, idx], qg[idx].astype(np.int64))
            np.add.at(want[:, 1], bins[ff, idx], qh[idx].astype(np.int64))
            np.add.at(want[:, 2], bins[ff, idx], 1)
            assert np.array_equal(h[ff], want)


def test_integer_subtraction_is_exact():
    n, f, nb = 4000, 5, 17
    bins, qg, qh = _data(n, f, nb, 3)
    left = np.nonzero(bins[2] <= 7)[0].astype(np.int32)
    right = np.nonzero(bins[2] > 7)[0].astype(np.int32)
    hp = O.hist_quantized(bins.ravel(), n, f, nb, qg, qh)
    hl = O.hist_quantized(bins.ravel(), n, f, nb, qg, qh, left)
    hr = O.hist_quantized(bins.ravel(), n, f, nb, qg, qh, right)
    assert np.array_equal(hp - hl, hr)


def _brute_split(hist, missing_bin, widths, gu, hu, l2, min_hess, min_data):
    """Every candidate's sums written as explicit bin sums (no running
    prefix), scored by quantized_split_gain; the winner is the largest gain,
    ties to the lowest (feature, bin, missing-left-before-right)."""
    nf, nb, _ = hist.shape
    hmin = int(np.ceil(min_hess * hu)) if min_hess > 0 else 0
    score = lambda g, h: (g / gu) ** 2 / (h / hu + l2)
    best = None
    for f in range(nf):
        tot = hist[f].sum(axis=0)
        mb = missing_bin[f]
        n_scan = mb if mb >= 0 else nb
        lim = min(n_scan, widths[f])
        miss = hist[f, mb] if mb >= 0 else np.zeros(3, np.int64)
        for b in range(lim):
            if b == n_scan - 1 and miss[2] == 0:
                break
            base = hist[f, :b + 1].sum(axis=0)
            cands = []
            if mb >= 0:
                cands.append((base + miss, 0))
            if mb < 0 or miss[2] > 0:
                cands.append((base, 1))
            for L, order in cands:
                R = tot - L
                if L[1] < hmin or R[1] < hmin or L[2] < min_data or R[2] < min_data:
                    continue
                g = score(L[0], L[1]) + score(R[0], R[1]) - score(tot[0], tot[1])
                if g > 0 and (best is None or g > best[0]):
                    best = (g, f, b, order == 0)
    return best


@pytest.mark.parametrize("seed", range(12))
def test_quantized_split_matches_brute_force(seed):
    rng = np.random.default_rng(100 + seed)
    nf, nb = 4, 9
    n = int(rng.integers(30, 400))
    bins = rng.integers(0, nb, size=(nf, n), dtype=np.uint8)
    qg = rng.integers(-2, 3, size=n).astype(np.int8)
    qh = rng.integers(0, 5, size=n).astype(np.int8)
    missing = np.full(nf, -1, np.int32)
    if seed % 3 == 1:
        missing[1] = nb - 1    # a reserved missing bin on feature 1
    if seed % 4 == 2:
        bins[0] = bins[0] % 4  # a narrow feature: width 4
    widths = np.array([max(int(bins[f].max()) + 1, missing[f] + 1) for f in range(nf)], np.int32)
    h = O.hist_quantized(bins.ravel(), n, nf, nb, qg, qh)
    gu, hu = 2.0 / 0.37, 4.0 / 0.25
    md = int(rng.integers(1, 12))
    found, f, b, dl, gain = O.split_quantized(h, missing, widths, gu, hu, 0.0, 1.0, 1e-3, md)
    want = _brute_split(h, missing, widths, gu, hu, 1.0, 1e-3, md)
    if want is None:
        assert not found
    else:
        assert found and (f, b, dl) == want[1:] and gain == pytest.approx(want[0], rel=1e-12)


def test_split_tie_prefers_lowest_feature_and_bin():
    """Two identical features: the first in scan order wins (strict '>')."""
    nb = 6
    h1 = np.array([[3, 8, 10], [5, 8, 10], [-4, 8, 10], [-6, 8, 10], [0, 8, 10], [0, 0, 0]],
                  np.int64)
    h = np.stack([h1, h1, h1])
    found, f, b, dl, g = O.split_quantized(h, np.full(3, -1, np.int32), np.full(3, nb, np.int32),
                                           1.0, 1.0, 0.0, 1.0, 1e-3, 1)
    assert found and f == 0 and b == 1


def _c2_like(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(10, n))
    logit = x[0] * x[1] + 0.8 * x[2] - 0.5 * x[3] * x[4] + 0.3 * x[5]
    y = (rng.uniform(size=n) < 1 / (1 + np.exp(-logit))).astype(np.float64)
    return x, y


def test_quantized_training_is_thread_count_invariant():
    n, f = 6000, 10
    x, y = _c2_like(n, 7)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=63)
    p1 = O.default_params(objective=1, num_iterations=6, num_leaves=15, use_quantized_grad=1,
                          n_threads=1)
    p8 = O.default_params(objective=1, num_iterations=6, num_leaves=15, use_quantized_grad=1,
                          n_threads=8)
    m1 = O.train(bins, n, f, 63, y, p1, missing_bin=mb)
    m8 = O.train(bins, n, f, 63, y, p8, missing_bin=mb)
    for k in ("feature", "threshold", "left", "right", "value", "default_left"):
        assert np.array_equal(getattr(m1, k), getattr(m8, k))
    assert np.array_equal(m1.train_raw(n), m8.train_raw(n))


def test_quantized_training_learns_like_float():
    n, f = 8000, 10
    x, y = _c2_like(n, 11)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=63)
    kw = dict(objective=1, num_iterations=30, num_leaves=15)
    mq = O.train(bins, n, f, 63, y, O.default_params(**kw, use_quantized_grad=1), missing_bin=mb)
    mf = O.train(bins, n, f, 63, y, O.default_params(**kw), missing_bin=mb)

    def logloss(m):
        raw = m.train_raw(n)
        p = 1 / (1 + np.exp(-raw))
        return -np.mean(y * np.log(p) + (1 - y) * np.log(1 - p))

    base = -np.mean(y * np.log(y.mean()) + (1 - y) * np.log(1 - y.mean()))
    lq, lf = logloss(mq), logloss(mf)
    assert lq < base - 0.05 and lf < base - 0.05
    assert abs(lq - lf) < 0.03
    # node covers add up: each internal node's count = children's counts
    for t in range(mq.n_trees):
        tr = mq.tree(t)
        for i in range(len(tr["feature"])):
            if tr["feature"][i] >= 0:
                assert tr["count"][i] == tr["count"][tr["left"][i]] + tr["count"][tr["right"][i]]
