"""sample_weight checks at the C ABI (boosting._check_sample_weight,
src/mojotrees/boosting.mojo:334-343): one finite, nonnegative weight per row
with a positive sum, refused before any device work, on any host."""
import ctypes as C

import numpy as np
import pytest

from mojoboost_amd import _lib
from mojoboost_amd._lib import lib, ptr


@pytest.mark.parametrize("w", [[1.0, -1.0, 1.0, 1.0], [1.0, np.nan, 1.0, 1.0], [0.0, 0.0, 0.0, 0.0],
                               [1.0, np.inf, 1.0, 1.0]])
def test_bad_sample_weights_are_refused(w):
    L = lib()
    e = L.mojotrees_error_create()
    x = np.arange(8, dtype=float)
    y = np.array([0.0, 1.0, 0.0, 1.0])
    h = C.c_void_p()
    wa = np.asarray(w, float)
    rc = L.mojotrees_train_dense(ptr(x), 4, 2, ptr(y), ptr(wa), b"objective=regression", C.byref(h), e)
    assert rc == _lib.ERROR_INVALID_ARGUMENT and h.value is None
    assert b"sample_weight" in L.mojotrees_error_message(e)
    L.mojotrees_error_free(e)


def test_estimator_checks_the_weight_length():
    from mojoboost_amd.sklearn import MojoTreesRegressor

    with pytest.raises(ValueError, match="sample_weight"):
        MojoTreesRegressor(n_estimators=1).fit(np.zeros((4, 2)), np.zeros(4), sample_weight=np.ones(3))
