"""The oracle against the reference's checked-in golden bit patterns.

tests/golden/golden_bits.json holds the literal IEEE-754 bits the reference
records in tests/test_golden_bits.mojo:322-7660 for its CPU fits (every
tree's structure and node values, every row's raw score and prediction).
The inputs are the closed-form generators of that file, restated in
tests/golden_fixtures.py. A match here pins, bit for bit: binning
(bin_equal_width, fit_bins + transform), the objectives, the base score and
the reference's own exp/log, the float histogram (including row blocks), the
split search, the leaf-wise grower, bagging, feature fraction, the softmax
loop, the score update and prediction; `misscat` adds missing-value routing
by each node's default direction and category-set splits together.
"""
import numpy as np
import pytest

import golden_fixtures as G
import oracle_lib as O

FIXTURES = ["l2", "logit", "multi", "bagged", "ffrac", "large", "misscat"]


def _bins_for(x, n, f, binning):
    """The fixture's binning: equal-width, fit_bins, or fit_bins with category
    tables (categorical.fit_categorical_spec, src/mojotrees/categorical.mojo:
    419-464: a feature's distinct codes, all kept when there are at most
    max_bins - 1, code c in bin 1 + its rank in ascending order)."""
    kind, nb = binning[0], binning[1]
    if kind == "equal":
        return O.bin_equal_width(x, n, f, nb), None, None
    bins, _, _, mb = O.fit_transform(x, n, f, max_bins=nb)
    if kind == "fit":
        return bins, mb, None
    ncat = np.zeros(f, np.int32)
    bins = bins.reshape(f, n).copy()
    for c in binning[2]:
        codes = np.unique(x[c * n:(c + 1) * n])
        assert len(codes) <= nb - 1
        bins[c] = 1 + np.searchsorted(codes, x[c * n:(c + 1) * n])
        ncat[c] = len(codes)
        mb[c] = -1
    return bins.ravel(), mb, ncat


@pytest.fixture(scope="module")
def gold():
    return G.load_golden()


@pytest.mark.parametrize("name", FIXTURES)
def test_golden_bits(name, gold):
    x, n, f, y, binning, kw = G.fixture(name)
    nb = binning[1]
    bins, mb, ncat = _bins_for(x, n, f, binning)
    p = O.default_params(**kw, n_threads=2)
    if ncat is not None:
        p.n_categories = ncat.ctypes.data  # ncat outlives the call
    model = O.train(bins, n, f, nb, y, p, missing_bin=mb)
    ints, vals, raw, pred = G.record(model, bins, n, f)
    want = gold[name]
    assert ints == want["ints"], "tree structure moved"
    assert vals == want["vals"], "node value bits moved"
    assert raw == want["raw"], "raw score bits moved"
    assert pred == want["pred"], "prediction bits moved"


def test_golden_detects_planted_fma_change(gold):
    """A plausible mistake (prediction sums without fused multiply-add) must
    fail the golden comparison."""
    x, n, f, y, (_, nb, *_), kw = G.fixture("l2")
    bins = O.bin_equal_width(x, n, f, nb)
    model = O.train(bins, n, f, nb, y, O.default_params(**kw, fused_predict=0))
    _, _, raw, _ = G.record(model, bins, n, f)
    assert raw != gold["l2"]["raw"]


def test_training_raw_equals_prediction():
    x, n, f, y, (_, nb, *_), kw = G.fixture("logit")
    bins = O.bin_equal_width(x, n, f, nb)
    model = O.train(bins, n, f, nb, y, O.default_params(**kw))
    raw, _ = model.predict_binned(bins, n, f)
    assert np.array_equal(model.train_raw(n), raw)
