"""scikit-learn-style estimators over the mojotrees C ABI.

Same names and call shapes as the reference's estimators
(python/mojotrees/sklearn.py: MojoTreesRegressor :5319, MojoTreesClassifier
:6178; fit :5548/:6412, predict :6016/:6898, predict_proba :6913, save/load
:6140-6162). Training goes through `mojotrees_train_dense` into the HIP
library (column-major float64 X by address, as bindings/_mojotrees.mojo:2102
takes it); device="gpu" never falls back to a CPU trainer.
"""
import ctypes as C

import numpy as np

from . import _lib
from ._lib import MojoTreesError, lib, ptr


class _Error:
    def __init__(self):
        self.h = lib().mojotrees_error_create()

    def message(self):
        m = lib().mojotrees_error_message(self.h)
        return m.decode(errors="replace") if m else ""

    def check(self, rc):
        if rc != _lib.OK:
            raise MojoTreesError(rc, self.message())

    def __del__(self):
        try:
            lib().mojotrees_error_free(self.h)
        except Exception:
            pass


def _feature_names(X):
    """Column names of a DataFrame-like X when every one is a string (the
    estimators' feature_names_in_, python/mojotrees/sklearn.py:4776-4830),
    else None."""
    cols = getattr(X, "columns", None)
    if cols is None:
        return None
    names = list(cols)
    if not names or not all(isinstance(c, str) for c in names):
        return None
    return np.asarray(names, dtype=object)


def _set_feature_names(est, X):
    names = _feature_names(X)
    if names is None:
        est.__dict__.pop("feature_names_in_", None)
    else:
        est.feature_names_in_ = names


def _colmajor(X):
    X = np.asarray(X, dtype=np.float64)
    if X.ndim != 2:
        raise ValueError("X must be 2-dimensional")
    return np.asfortranarray(X), X.shape[0], X.shape[1]


def _predict_device(device):
    if device is None or device == "cpu":
        return _lib.DEVICE_CPU
    if device == "gpu":
        return _lib.DEVICE_GPU
    if device == "auto":
        return _lib.DEVICE_AUTO
    raise ValueError(f"device must be None, 'cpu', 'gpu' or 'auto', not {device!r}")


class _Booster:
    """An owned model handle."""

    def __init__(self, handle):
        self.h = handle

    def __del__(self):
        try:
            if self.h:
                lib().mojotrees_model_free(self.h)
        except Exception:
            pass

    def _count(self, fn):
        v = C.c_int64()
        e = _Error()
        e.check(getattr(lib(), fn)(self.h, C.byref(v), e.h))
        return int(v.value)

    @property
    def num_features(self):
        return self._count("mojotrees_model_num_features")

    @property
    def num_classes(self):
        return self._count("mojotrees_model_num_classes")

    @property
    def num_trees(self):
        return self._count("mojotrees_model_num_trees")

    @property
    def num_iterations(self):
        return self._count("mojotrees_model_num_iterations")

    def predict(self, X, raw=False, start_iteration=0, num_iteration=0, device=None):
        Xf, n, f = _colmajor(X)
        k = self.num_classes
        out = np.zeros(n * k)
        e = _Error()
        flags = _lib.PREDICT_RAW if raw else _lib.PREDICT_RESPONSE
        e.check(lib().mojotrees_predict_ex(self.h, ptr(Xf.ravel(order="K")), n, f,
                                           start_iteration, num_iteration or 0, flags,
                                           _predict_device(device), ptr(out), out.size, e.h))
        return out.reshape(n, k) if k > 1 else out

    def save(self, path, feature_names=None):
        """The v4 model file; with feature_names, its optional
        feature_names section (serialize.save_model,
        src/mojotrees/serialize.mojo:999-1030)."""
        e = _Error()
        if feature_names is None or len(feature_names) == 0:
            e.check(lib().mojotrees_save_model(self.h, str(path).encode(), e.h))
            return
        enc = [str(nm).encode() for nm in feature_names]
        arr = (C.c_char_p * len(enc))(*enc)
        e.check(lib().mbh_save_model_named(self.h, str(path).encode(), C.cast(arr, C.c_void_p),
                                           len(enc), e.h))

    @staticmethod
    def load(path):
        h = C.c_void_p()
        e = _Error()
        e.check(lib().mojotrees_load_model(str(path).encode(), C.byref(h), e.h))
        return _Booster(h)

    @staticmethod
    def feature_names(path):
        """The names a model file carries (serialize.load_feature_names),
        [] when it has none."""
        out = C.c_void_p()
        cnt = C.c_int64()
        e = _Error()
        e.check(lib().mbh_model_feature_names(str(path).encode(), C.byref(out), C.byref(cnt), e.h))
        if not out.value:
            return []
        try:
            names, at = [], out.value
            for _ in range(cnt.value):
                raw = C.string_at(at)
                names.append(raw.decode())
                at += len(raw) + 1
            return names
        finally:
            lib().mojotrees_string_free(C.cast(out, C.c_char_p))

    def dump_json(self):
        out = C.c_char_p()
        e = _Error()
        e.check(lib().mojotrees_model_dump_json(self.h, C.byref(out), e.h))
        try:
            return out.value.decode()
        finally:
            lib().mojotrees_string_free(out)

    def feature_importance(self, importance_type="split"):
        t = _lib.IMPORTANCE_GAIN if importance_type == "gain" else _lib.IMPORTANCE_SPLIT
        out = np.zeros(self.num_features)
        e = _Error()
        e.check(lib().mojotrees_feature_importance(self.h, t, ptr(out), out.size, e.h))
        return out


def _train(X, y, params: str, sample_weight=None):
    Xf, n, f = _colmajor(X)
    y = np.ascontiguousarray(y, dtype=np.float64)
    if y.shape[0] != n:
        raise ValueError("y must have one entry per row of X")
    w = None
    if sample_weight is not None:
        w = np.ascontiguousarray(sample_weight, dtype=np.float64)
        if w.shape != (n,):
            raise ValueError("sample_weight length must equal n_rows")
    h = C.c_void_p()
    e = _Error()
    e.check(lib().mojotrees_train_dense(ptr(Xf.ravel(order="K")), n, f, ptr(y), ptr(w),
                                        params.encode(), C.byref(h), e.h))
    return _Booster(h)


class _Base:
    _objective = "regression"

    def __init__(self, n_estimators=100, learning_rate=0.1, num_leaves=31, max_depth=-1,
                 min_child_samples=20, min_child_weight=1e-3, reg_alpha=0.0, reg_lambda=1.0,
                 colsample_bytree=1.0, subsample=1.0, subsample_freq=0, max_bin=255,
                 random_state=None, device="gpu", use_quantized_grad=False,
                 num_grad_quant_bins=4, stochastic_rounding=True, categorical_feature=None,
                 max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=10.0, cat_l2=10.0,
                 min_data_per_group=100):
        self.n_estimators = n_estimators
        self.learning_rate = learning_rate
        self.num_leaves = num_leaves
        self.max_depth = max_depth
        self.min_child_samples = min_child_samples
        self.min_child_weight = min_child_weight
        self.reg_alpha = reg_alpha
        self.reg_lambda = reg_lambda
        self.colsample_bytree = colsample_bytree
        self.subsample = subsample
        self.subsample_freq = subsample_freq
        self.max_bin = max_bin
        self.random_state = random_state
        self.device = device
        self.use_quantized_grad = use_quantized_grad
        self.num_grad_quant_bins = num_grad_quant_bins
        self.stochastic_rounding = stochastic_rounding
        # categorical_feature: column indices split by category set
        # (LightGBM's parameter; the reference's estimators,
        # python/mojotrees/sklearn.py:929-951), with LightGBM's defaults
        self.categorical_feature = categorical_feature
        self.max_cat_to_onehot = max_cat_to_onehot
        self.max_cat_threshold = max_cat_threshold
        self.cat_smooth = cat_smooth
        self.cat_l2 = cat_l2
        self.min_data_per_group = min_data_per_group
        self.booster_ = None

    def _params(self, extra=""):
        if self.device not in ("gpu", "auto", "cpu"):
            raise ValueError("device must be 'gpu', 'auto' or 'cpu'")
        p = [f"objective={self._objective}", f"num_iterations={self.n_estimators}",
             f"learning_rate={self.learning_rate!r}", f"num_leaves={self.num_leaves}",
             f"max_depth={self.max_depth}", f"min_data_in_leaf={self.min_child_samples}",
             f"min_sum_hessian_in_leaf={self.min_child_weight!r}",
             f"lambda_l1={self.reg_alpha!r}", f"lambda_l2={self.reg_lambda!r}",
             f"feature_fraction={self.colsample_bytree!r}",
             f"bagging_fraction={self.subsample!r}", f"bagging_freq={self.subsample_freq}",
             f"max_bin={self.max_bin}", f"device={self.device}",
             f"use_quantized_grad={'true' if self.use_quantized_grad else 'false'}",
             f"num_grad_quant_bins={self.num_grad_quant_bins}",
             f"stochastic_rounding={'true' if self.stochastic_rounding else 'false'}"]
        if self.random_state is not None:
            p += [f"feature_fraction_seed={int(self.random_state)}",
                  f"bagging_seed={int(self.random_state)}"]
        cats = self.categorical_feature
        if cats is not None and not (isinstance(cats, str) and cats == "auto"):
            if isinstance(cats, (str, bytes)):
                raise ValueError("categorical_feature must be None, 'auto' or a sequence of column indices")
            idx = []
            for c in cats:
                if isinstance(c, bool) or int(c) != c or int(c) < 0:
                    raise ValueError(f"categorical_feature entry {c!r} is not a column index")
                if int(c) in idx:
                    raise ValueError(f"categorical_feature lists feature {int(c)} twice")
                idx.append(int(c))
            if idx:
                p += ["categorical_feature=" + ",".join(str(i) for i in sorted(idx)),
                      f"max_cat_to_onehot={self.max_cat_to_onehot}",
                      f"max_cat_threshold={self.max_cat_threshold}",
                      f"cat_smooth={self.cat_smooth!r}", f"cat_l2={self.cat_l2!r}",
                      f"min_data_per_group={self.min_data_per_group}"]
        return " ".join(p) + (" " + extra if extra else "")

    def save(self, path):
        """v4 model file, with feature_names_in_ as its feature_names section
        when the estimator was fitted on named columns (the reference's
        estimators, python/mojotrees/sklearn.py:6140-6148)."""
        self._check_fitted()
        self.booster_.save(path, getattr(self, "feature_names_in_", None))

    def _restore(self, path):
        self.booster_ = _Booster.load(path)
        names = _Booster.feature_names(path)
        if names:
            self.feature_names_in_ = np.asarray(names, dtype=object)

    def _check_fitted(self):
        if self.booster_ is None:
            raise RuntimeError("estimator is not fitted")

    @property
    def n_features_in_(self):
        self._check_fitted()
        return self.booster_.num_features

    def feature_importances(self, importance_type="split"):
        self._check_fitted()
        return self.booster_.feature_importance(importance_type)


class MojoTreesRegressor(_Base):
    _objective = "regression"

    def fit(self, X, y, sample_weight=None):
        self.booster_ = _train(X, y, self._params(), sample_weight)
        _set_feature_names(self, X)
        return self

    def predict(self, X, raw_score=False, start_iteration=0, num_iteration=None, device=None):
        """`device` as in the reference (python/mojotrees/sklearn.py:6016-6060):
        None predicts on the CPU, "gpu" on the device (an error without one),
        "auto" by the library's rule. Both give the same scores."""
        self._check_fitted()
        return self.booster_.predict(X, raw=raw_score, start_iteration=start_iteration,
                                     num_iteration=num_iteration, device=device)

    @classmethod
    def load(cls, path):
        est = cls()
        est._restore(path)
        return est


class MojoTreesClassifier(_Base):
    """Binary (logistic) for two classes, softmax multiclass for more; class
    labels are mapped to 0..K-1 in sorted order, as the reference's
    classifier does (python/mojotrees/sklearn.py:6412)."""
    _objective = "binary"

    def fit(self, X, y, sample_weight=None):
        y = np.asarray(y)
        self.classes_, yi = np.unique(y, return_inverse=True)
        k = len(self.classes_)
        if k < 2:
            raise ValueError("y needs at least two classes")
        if k == 2:
            self.booster_ = _train(X, yi.astype(np.float64), self._params(), sample_weight)
        else:
            params = self._params().replace("objective=binary", "objective=multiclass")
            self.booster_ = _train(X, yi.astype(np.float64), params + f" num_class={k}", sample_weight)
        _set_feature_names(self, X)
        return self

    def predict_proba(self, X, start_iteration=0, num_iteration=None, device=None):
        self._check_fitted()
        p = self.booster_.predict(X, start_iteration=start_iteration, num_iteration=num_iteration,
                                  device=device)
        if self.booster_.num_classes == 1:
            return np.column_stack([1.0 - p, p])
        return p.reshape(-1, self.booster_.num_classes)

    def predict(self, X, start_iteration=0, num_iteration=None, device=None):
        return self.classes_[np.argmax(self.predict_proba(X, start_iteration, num_iteration, device),
                                       axis=1)]

    def decision_function(self, X, start_iteration=0, num_iteration=None, device=None):
        self._check_fitted()
        raw = self.booster_.predict(X, raw=True, start_iteration=start_iteration,
                                    num_iteration=num_iteration, device=device)
        k = self.booster_.num_classes
        return raw if k == 1 else raw.reshape(-1, k)

    @classmethod
    def load(cls, path):
        est = cls()
        est._restore(path)
        k = est.booster_.num_classes
        est.classes_ = np.arange(2 if k == 1 else k)
        return est


class MojoTreesRanker(_Base):
    """LambdaRank learning to rank (the reference's MojoTreesRanker,
    python/mojotrees/sklearn.py:6951; objective lambdarank,
    src/mojotrees/ranking.mojo). fit takes LightGBM's `group`: one row count
    per query, in row order. Predictions are raw scores; only their order
    within a query means anything."""
    _objective = "lambdarank"

    def __init__(self, n_estimators=100, learning_rate=0.1, num_leaves=31, max_depth=-1,
                 min_child_samples=20, min_child_weight=1e-3, reg_alpha=0.0, reg_lambda=1.0,
                 colsample_bytree=1.0, subsample=1.0, subsample_freq=0, max_bin=255,
                 random_state=None, device="gpu",
                 use_quantized_grad=False, num_grad_quant_bins=4, stochastic_rounding=True,
                 lambdarank_truncation_level=30, sigmoid=1.0, lambdarank_norm=True):
        super().__init__(n_estimators=n_estimators, learning_rate=learning_rate,
                         num_leaves=num_leaves, max_depth=max_depth,
                         min_child_samples=min_child_samples, min_child_weight=min_child_weight,
                         reg_alpha=reg_alpha, reg_lambda=reg_lambda,
                         colsample_bytree=colsample_bytree, subsample=subsample,
                         subsample_freq=subsample_freq, max_bin=max_bin,
                         random_state=random_state, device=device,
                         use_quantized_grad=use_quantized_grad,
                         num_grad_quant_bins=num_grad_quant_bins,
                         stochastic_rounding=stochastic_rounding)
        self.lambdarank_truncation_level = lambdarank_truncation_level
        self.sigmoid = sigmoid
        self.lambdarank_norm = lambdarank_norm

    def fit(self, X, y, group, sample_weight=None):
        """subsample / subsample_freq bag whole queries
        (ranking._refresh_query_bag, src/mojotrees/ranking.mojo:667-686);
        sample_weight scales each row's lambda and hessian."""
        Xf, n, f = _colmajor(X)
        y = np.ascontiguousarray(y, dtype=np.float64)
        if y.shape[0] != n:
            raise ValueError("y must have one entry per row of X")
        w = None
        if sample_weight is not None:
            w = np.ascontiguousarray(sample_weight, dtype=np.float64)
            if w.shape != (n,):
                raise ValueError("sample_weight length must equal n_rows")
        g = np.ascontiguousarray(group, dtype=np.int32)
        if g.ndim != 1 or g.size == 0:
            raise ValueError("group must be a non-empty 1-d array of query sizes")
        params = self._params(
            f"lambdarank_truncation_level={self.lambdarank_truncation_level} "
            f"sigmoid={self.sigmoid!r} "
            f"lambdarank_norm={'true' if self.lambdarank_norm else 'false'}")
        h = C.c_void_p()
        e = _Error()
        e.check(lib().mbh_train_ranker_dense(ptr(Xf.ravel(order="K")), n, f, ptr(y), ptr(w), ptr(g), g.size,
                                             params.encode(), C.byref(h), e.h))
        self.booster_ = _Booster(h)
        _set_feature_names(self, X)
        return self

    def predict(self, X, start_iteration=0, num_iteration=None, device=None):
        self._check_fitted()
        return self.booster_.predict(X, raw=True, start_iteration=start_iteration,
                                     num_iteration=num_iteration, device=device)

    @classmethod
    def load(cls, path):
        est = cls()
        est._restore(path)
        return est
