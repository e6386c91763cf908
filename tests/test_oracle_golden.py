"""The oracle against the reference's checked-in golden bit patterns.

tests/golden/golden_bits.json holds the literal IEEE-754 bits the reference
records in tests/test_golden_bits.mojo:322-7660 for its CPU fits (every
tree's structure and node values, every row's raw score and prediction).
The inputs are the closed-form generators of that file, restated in
tests/golden_fixtures.py. A match here pins, bit for bit: binning
(bin_equal_width, fit_bins + transform), the objectives, the base score and
the reference's own exp/log, the float histogram (including row blocks), the
split search, the leaf-wise grower, bagging, feature fraction, the softmax
loop, the score update and prediction. `misscat` needs categorical set
splits, which are out of this build's scope, and is not run.
"""
import numpy as np
import pytest

import golden_fixtures as G
import oracle_lib as O

FIXTURES = ["l2", "logit", "multi", "bagged", "ffrac", "large"]


@pytest.fixture(scope="module")
def gold():
    return G.load_golden()


@pytest.mark.parametrize("name", FIXTURES)
def test_golden_bits(name, gold):
    x, n, f, y, (kind, nb), kw = G.fixture(name)
    if kind == "equal":
        bins = O.bin_equal_width(x, n, f, nb)
        mb = None
    else:
        bins, _, _, mb = O.fit_transform(x, n, f, max_bins=nb)
    model = O.train(bins, n, f, nb, y, O.default_params(**kw, n_threads=2), missing_bin=mb)
    ints, vals, raw, pred = G.record(model, bins, n, f)
    want = gold[name]
    assert ints == want["ints"], "tree structure moved"
    assert vals == want["vals"], "node value bits moved"
    assert raw == want["raw"], "raw score bits moved"
    assert pred == want["pred"], "prediction bits moved"


def test_golden_detects_planted_fma_change(gold):
    """A plausible mistake (prediction sums without fused multiply-add) must
    fail the golden comparison."""
    x, n, f, y, (_, nb), kw = G.fixture("l2")
    bins = O.bin_equal_width(x, n, f, nb)
    model = O.train(bins, n, f, nb, y, O.default_params(**kw, fused_predict=0))
    _, _, raw, _ = G.record(model, bins, n, f)
    assert raw != gold["l2"]["raw"]


def test_training_raw_equals_prediction():
    x, n, f, y, (_, nb), kw = G.fixture("logit")
    bins = O.bin_equal_width(x, n, f, nb)
    model = O.train(bins, n, f, nb, y, O.default_params(**kw))
    raw, _ = model.predict_binned(bins, n, f)
    assert np.array_equal(model.train_raw(n), raw)
