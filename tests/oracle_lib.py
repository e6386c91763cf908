"""ctypes binding to the CPU oracle (oracle/_build/liboracle.so).

Test infrastructure only: the oracle is the parity checker and the CPU
baseline, never part of the product path.
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = ROOT / "oracle" / "_build" / "liboracle.so"

OBJ_L2, OBJ_BINARY, OBJ_MULTICLASS, OBJ_LAMBDARANK = 0, 1, 2, 3


class Params(C.Structure):
    _fields_ = [
        ("objective", C.c_int32),
        ("num_class", C.c_int32),
        ("num_iterations", C.c_int32),
        ("learning_rate", C.c_double),
        ("num_leaves", C.c_int32),
        ("min_data_in_leaf", C.c_int32),
        ("lambda_l2", C.c_double),
        ("lambda_l1", C.c_double),
        ("min_sum_hessian", C.c_double),
        ("max_depth", C.c_int32),
        ("feature_fraction", C.c_double),
        ("feature_fraction_seed", C.c_int32),
        ("bagging_fraction", C.c_double),
        ("bagging_freq", C.c_int32),
        ("bagging_seed", C.c_int32),
        ("use_quantized_grad", C.c_int32),
        ("num_grad_quant_bins", C.c_int32),
        ("stochastic_rounding", C.c_int32),
        ("quant_seed", C.c_int32),
        ("goss", C.c_int32),
        ("top_rate", C.c_double),
        ("other_rate", C.c_double),
        ("goss_seed", C.c_int32),
        ("n_threads", C.c_int32),
        ("fused_score_update", C.c_int32),
        ("fused_predict", C.c_int32),
        ("totals_tree_reduce", C.c_int32),
        ("use_init_base", C.c_int32),
        ("init_base", C.c_double),
        ("query_starts", C.c_void_p),
        ("n_queries", C.c_int64),
        ("lambdarank_truncation_level", C.c_int32),
        ("lambdarank_norm", C.c_int32),
        ("lambdarank_sigmoid", C.c_double),
        ("n_categories", C.c_void_p),
        ("max_cat_to_onehot", C.c_int32),
        ("max_cat_threshold", C.c_int32),
        ("cat_smooth", C.c_double),
        ("cat_l2", C.c_double),
        ("min_data_per_group", C.c_int32),
        ("one_hot_max_size", C.c_int32),
        ("weights", C.c_void_p),
        ("quant_scale_rule", C.c_int32),
    ]


def _threads():
    """Oracle worker threads: the CPUs this process may use, at most 16 (a
    GPU box's CPU share for one GPU, whatever the host reports)."""
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def default_params(**kw) -> Params:
    p = Params(
        objective=OBJ_L2, num_class=1, num_iterations=100, learning_rate=0.1,
        num_leaves=31, min_data_in_leaf=20, lambda_l2=1.0, lambda_l1=0.0,
        min_sum_hessian=1e-3, max_depth=-1, feature_fraction=1.0,
        feature_fraction_seed=2, bagging_fraction=1.0, bagging_freq=0,
        bagging_seed=3, use_quantized_grad=0, num_grad_quant_bins=4,
        stochastic_rounding=1, quant_seed=11, goss=0, top_rate=0.2,
        other_rate=0.1, goss_seed=3, n_threads=_threads(), fused_score_update=1,
        fused_predict=1, totals_tree_reduce=1, use_init_base=0, init_base=0.0,
        query_starts=None, n_queries=0, lambdarank_truncation_level=30, lambdarank_norm=1,
        lambdarank_sigmoid=1.0, n_categories=None, max_cat_to_onehot=4, max_cat_threshold=32,
        cat_smooth=10.0, cat_l2=10.0, min_data_per_group=100, one_hot_max_size=-1, weights=None,
        quant_scale_rule=0,
    )
    for k, v in kw.items():
        setattr(p, k, v)
    return p


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        P = C.POINTER
        L.orc_splitmix64.restype = C.c_uint64
        L.orc_splitmix64.argtypes = [C.c_uint64]
        L.orc_uniform.restype = C.c_double
        L.orc_uniform.argtypes = [C.c_uint64]
        L.orc_exp.restype = C.c_double
        L.orc_exp.argtypes = [C.c_double]
        L.orc_log.restype = C.c_double
        L.orc_log.argtypes = [C.c_double]
        L.orc_sigmoid.restype = C.c_double
        L.orc_sigmoid.argtypes = [C.c_double]
        L.orc_quant_stream.restype = C.c_uint64
        L.orc_quant_stream.argtypes = [C.c_int64] * 4
        L.orc_train.restype = C.c_void_p
        L.orc_train.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_void_p,
                                C.c_void_p, P(Params), C.c_char_p, C.c_int32]
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_model_num_trees.restype = C.c_int32
        L.orc_model_num_trees.argtypes = [C.c_void_p]
        L.orc_model_num_class.restype = C.c_int32
        L.orc_model_num_class.argtypes = [C.c_void_p]
        L.orc_model_total_nodes.restype = C.c_int64
        L.orc_model_total_nodes.argtypes = [C.c_void_p]
        L.orc_model_arrays.argtypes = [C.c_void_p] + [C.c_void_p] * 11
        L.orc_model_train_raw.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_model_round_seconds.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_predict_binned.restype = C.c_int32
        L.orc_predict_binned.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int32,
                                         C.c_void_p, C.c_void_p]
        L.orc_bin_equal_width.restype = C.c_int32
        L.orc_bin_equal_width.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_void_p]
        L.orc_fit_bins.restype = C.c_int32
        L.orc_fit_bins.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_int32,
                                   C.c_int32, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                   C.c_void_p]
        L.orc_transform.restype = C.c_int32
        L.orc_transform.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_grad_hess.restype = C.c_int32
        L.orc_grad_hess.argtypes = [C.c_int32, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32,
                                    C.c_int32, C.c_void_p, C.c_void_p]
        L.orc_quantize.restype = C.c_int32
        L.orc_quantize.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64,
                                   C.c_int32, C.c_int32, C.c_int64, C.c_int64, C.c_int64,
                                   C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_quantize_rule.restype = C.c_int32
        L.orc_quantize_rule.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64,
                                        C.c_int32, C.c_int32, C.c_int64, C.c_int64, C.c_int64,
                                        C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_magnitude_sums.restype = C.c_int32
        L.orc_magnitude_sums.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p,
                                         C.c_void_p]
        L.orc_largest_power_of_two_at_most.restype = C.c_double
        L.orc_largest_power_of_two_at_most.argtypes = [C.c_double]
        L.orc_fixed_point_scale_pow2.restype = C.c_double
        L.orc_fixed_point_scale_pow2.argtypes = [C.c_double]
        L.orc_hist_quantized32.restype = C.c_int32
        L.orc_hist_quantized32.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32,
                                           C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                           C.c_void_p]
        L.orc_hist_quantized.restype = C.c_int32
        L.orc_hist_quantized.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32,
                                         C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                         C.c_void_p]
        L.orc_hist_float.restype = C.c_int32
        L.orc_hist_float.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_void_p,
                                     C.c_void_p]
        L.orc_split_quantized.restype = C.c_int32
        L.orc_split_quantized.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                          C.c_void_p, C.c_double, C.c_double, C.c_double,
                                          C.c_double, C.c_double, C.c_int32, C.c_void_p,
                                          C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_lambdarank.restype = C.c_int32
        L.orc_lambdarank.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32,
                                     C.c_double, C.c_int32, C.c_void_p, C.c_void_p]
        L.orc_log2.restype = C.c_double
        L.orc_log2.argtypes = [C.c_double]
        L.orc_goss_select.restype = C.c_int32
        L.orc_goss_select.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_double, C.c_double,
                                      C.c_int32, C.c_int64, C.c_void_p, C.c_void_p,
                                      P(C.c_int64)]
        L.orc_model_cat_bits.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_grad_hess_w.restype = C.c_int32
        L.orc_grad_hess_w.argtypes = [C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                      C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]
        L.orc_cat_split.restype = C.c_int32
        L.orc_cat_split.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_double, C.c_double,
                                    C.c_int64, C.c_double, C.c_double, C.c_double, C.c_int32,
                                    C.c_int32, C.c_int32, C.c_double, C.c_double, C.c_int32,
                                    C.c_int32, C.c_void_p, C.c_void_p]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Model:
    """Flat-array view of an oracle model."""

    def __init__(self, handle):
        L = lib()
        self.h = handle
        self.n_trees = L.orc_model_num_trees(handle)
        self.num_class = L.orc_model_num_class(handle)
        nn = L.orc_model_total_nodes(handle)
        self.base = np.zeros(self.num_class)
        self.off = np.zeros(self.n_trees + 1, np.int64)
        i32 = lambda: np.zeros(nn, np.int32)
        f64 = lambda: np.zeros(nn, np.float64)
        self.feature, self.threshold, self.left, self.right = i32(), i32(), i32(), i32()
        self.value, self.default_left, self.missing_bin = f64(), i32(), i32()
        self.gain, self.count = f64(), f64()
        L.orc_model_arrays(handle, _ptr(self.base), _ptr(self.off), _ptr(self.feature),
                           _ptr(self.threshold), _ptr(self.left), _ptr(self.right),
                           _ptr(self.value), _ptr(self.default_left), _ptr(self.missing_bin),
                           _ptr(self.gain), _ptr(self.count))
        self.cat_bits = np.zeros((nn, 4), np.uint64)
        L.orc_model_cat_bits(handle, _ptr(self.cat_bits))

    def tree(self, t):
        a, b = self.off[t], self.off[t + 1]
        return {k: getattr(self, k)[a:b] for k in
                ("feature", "threshold", "left", "right", "value", "default_left",
                 "missing_bin", "gain", "count")}

    def train_raw(self, n_rows):
        out = np.zeros(n_rows * self.num_class)
        lib().orc_model_train_raw(self.h, _ptr(out))
        return out

    def round_seconds(self, n_iter):
        out = np.zeros(n_iter)
        lib().orc_model_round_seconds(self.h, _ptr(out))
        return out

    def predict_binned(self, bins_cm, n_rows, n_features):
        raw = np.zeros(n_rows * self.num_class)
        resp = np.zeros(n_rows * self.num_class)
        lib().orc_predict_binned(self.h, _ptr(bins_cm), n_rows, n_features, _ptr(raw), _ptr(resp))
        return raw, resp

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.orc_model_free(self.h)
            self.h = None


def train(bins_cm, n_rows, n_features, n_bins, labels, params, missing_bin=None):
    bins_cm = np.ascontiguousarray(bins_cm, dtype=np.uint8)
    labels = np.ascontiguousarray(labels, dtype=np.float64)
    mb = None if missing_bin is None else np.ascontiguousarray(missing_bin, dtype=np.int32)
    err = C.create_string_buffer(512)
    h = lib().orc_train(_ptr(bins_cm), n_rows, n_features, n_bins, _ptr(mb), _ptr(labels),
                        C.byref(params), err, 512)
    if not h:
        raise RuntimeError("oracle training failed: " + err.value.decode())
    return Model(h)


def bin_equal_width(x_cm, n_rows, n_features, n_bins):
    out = np.zeros(n_rows * n_features, np.uint8)
    rc = lib().orc_bin_equal_width(_ptr(np.ascontiguousarray(x_cm, np.float64)), n_rows,
                                   n_features, n_bins, _ptr(out))
    assert rc == 0
    return out


def fit_transform(x_cm, n_rows, n_features, max_bins=255, min_data_in_bin=3, use_missing=1,
                  sample_cnt=200_000, seed=1):
    x_cm = np.ascontiguousarray(x_cm, np.float64)
    edges = np.zeros(n_features * max_bins)
    n_edges = np.zeros(n_features, np.int32)
    mb = np.zeros(n_features, np.int32)
    rc = lib().orc_fit_bins(_ptr(x_cm), n_rows, n_features, max_bins, min_data_in_bin,
                            use_missing, sample_cnt, seed, _ptr(edges), _ptr(n_edges), _ptr(mb))
    assert rc == 0, rc
    bins = np.zeros(n_rows * n_features, np.uint8)
    lib().orc_transform(_ptr(x_cm), n_rows, n_features, max_bins, _ptr(edges), _ptr(n_edges),
                        _ptr(mb), _ptr(bins))
    return bins, edges.reshape(n_features, max_bins), n_edges, mb


def grad_hess(objective, raw, labels, num_class=1, class_k=0):
    n = len(labels)
    g = np.zeros(n)
    h = np.zeros(n)
    lib().orc_grad_hess(objective, _ptr(np.ascontiguousarray(raw, np.float64)),
                        _ptr(np.ascontiguousarray(labels, np.float64)), n, num_class, class_k,
                        _ptr(g), _ptr(h))
    return g, h


def grad_hess_w(objective, raw, labels, weights, num_class=1, class_k=0):
    n = len(labels)
    g = np.zeros(n)
    h = np.zeros(n)
    lib().orc_grad_hess_w(objective, _ptr(np.ascontiguousarray(raw, np.float64)),
                          _ptr(np.ascontiguousarray(labels, np.float64)),
                          _ptr(np.ascontiguousarray(weights, np.float64)), n, num_class, class_k,
                          _ptr(g), _ptr(h))
    return g, h


def quantize(grad, hess, rows=None, quant_bins=4, stochastic=1, seed=11, round_index=0,
             class_index=0, const_hessian=0):
    n = len(grad)
    qg = np.zeros(n, np.int8)
    qh = np.zeros(n, np.int8)
    sc = np.zeros(4)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    lib().orc_quantize(_ptr(np.ascontiguousarray(grad, np.float64)),
                       _ptr(np.ascontiguousarray(hess, np.float64)), n, _ptr(r),
                       0 if r is None else len(r), quant_bins, stochastic, seed, round_index,
                       class_index, const_hessian, _ptr(qg), _ptr(qh), _ptr(sc))
    return qg, qh, sc


RULE_MAX_ABS, RULE_MAGNITUDE_SUM = 0, 1


def quantize_rule(grad, hess, rule, rows=None, quant_bins=4, stochastic=1, seed=11,
                  round_index=0, class_index=0, const_hessian=0):
    """Either lattice, int32 values: (qg, qh, [gu, hu, gmax, hmax]); raises
    when the magnitudes are out of the fixed-point range."""
    n = len(grad)
    qg = np.zeros(n, np.int32)
    qh = np.zeros(n, np.int32)
    sc = np.zeros(4)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    rc = lib().orc_quantize_rule(_ptr(np.ascontiguousarray(grad, np.float64)),
                                 _ptr(np.ascontiguousarray(hess, np.float64)), n, _ptr(r),
                                 0 if r is None else len(r), quant_bins, stochastic, seed,
                                 round_index, class_index, const_hessian, rule, _ptr(qg), _ptr(qh),
                                 _ptr(sc))
    if rc != 0:
        raise ValueError("magnitudes out of range for the fixed-point lattice")
    return qg, qh, sc


def magnitude_sums(grad, hess, in_sample=None):
    out = np.zeros(2)
    m = None if in_sample is None else np.ascontiguousarray(in_sample, np.uint8)
    lib().orc_magnitude_sums(_ptr(np.ascontiguousarray(grad, np.float64)),
                             _ptr(np.ascontiguousarray(hess, np.float64)), len(grad), _ptr(m),
                             _ptr(out))
    return float(out[0]), float(out[1])


def largest_power_of_two_at_most(x):
    return float(lib().orc_largest_power_of_two_at_most(x))


def fixed_point_scale_pow2(total):
    return float(lib().orc_fixed_point_scale_pow2(total))


def hist_quantized32(bins_cm, n_rows, n_features, n_bins, qg, qh, rows=None):
    out = np.zeros(n_features * n_bins * 3, np.int64)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    lib().orc_hist_quantized32(_ptr(np.ascontiguousarray(bins_cm, np.uint8)), n_rows,
                               n_features, n_bins, _ptr(np.ascontiguousarray(qg, np.int32)),
                               _ptr(np.ascontiguousarray(qh, np.int32)), _ptr(r),
                               0 if r is None else len(r), _ptr(out))
    return out.reshape(n_features, n_bins, 3)


def hist_quantized(bins_cm, n_rows, n_features, n_bins, qg, qh, rows=None):
    out = np.zeros(n_features * n_bins * 3, np.int64)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    lib().orc_hist_quantized(_ptr(np.ascontiguousarray(bins_cm, np.uint8)), n_rows,
                             n_features, n_bins, _ptr(np.ascontiguousarray(qg, np.int8)),
                             _ptr(np.ascontiguousarray(qh, np.int8)), _ptr(r),
                             0 if r is None else len(r), _ptr(out))
    return out.reshape(n_features, n_bins, 3)


def split_quantized(hist, missing_bin, widths, gu, hu, l1=0.0, l2=1.0, min_hess=1e-3,
                    min_data=20):
    nf, nb, _ = hist.shape
    of, ob, odl = C.c_int32(), C.c_int32(), C.c_int32()
    og = C.c_double()
    mb = np.ascontiguousarray(missing_bin, np.int32)
    w = None if widths is None else np.ascontiguousarray(widths, np.int32)
    found = lib().orc_split_quantized(_ptr(np.ascontiguousarray(hist, np.int64)), nf, nb,
                                      _ptr(mb), _ptr(w), gu, hu, l1, l2, min_hess, min_data,
                                      C.byref(of), C.byref(ob), C.byref(odl), C.byref(og))
    return bool(found), of.value, ob.value, bool(odl.value), og.value


def goss_select(grad, hess, top_rate=0.2, other_rate=0.1, seed=3, round_index=0):
    """One GOSS selection (no warmup): (rows, scale, scaled grad, scaled hess)."""
    g = np.array(grad, np.float64)
    h = np.array(hess, np.float64)
    n = len(g)
    rows = np.zeros(n, np.int32)
    scale = np.zeros(n)
    cnt = C.c_int64(0)
    rc = lib().orc_goss_select(_ptr(g), _ptr(h), n, top_rate, other_rate, seed, round_index,
                               _ptr(rows), _ptr(scale), C.byref(cnt))
    assert rc == 0, rc
    return rows[:cnt.value], scale[:cnt.value], g, h


def goss_select_multiclass(prob, labels, K, top_rate=0.2, other_rate=0.1, seed=3, round_index=0,
                           weights=None):
    """One multiclass round's GOSS sample (no warmup) from row-major class
    probabilities: (rows, other flags per row, multiplier)."""
    L = lib()
    L.orc_goss_select_multiclass.restype = C.c_int32
    L.orc_goss_select_multiclass.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_void_p,
                                             C.c_double, C.c_double, C.c_int32, C.c_int64, C.c_void_p,
                                             C.c_void_p, C.c_void_p, C.c_void_p]
    pr = np.ascontiguousarray(prob, np.float64).ravel()
    y = np.ascontiguousarray(labels, np.float64)
    n = len(y)
    w = None if weights is None else np.ascontiguousarray(weights, np.float64)
    rows = np.zeros(n, np.int32)
    other = np.zeros(n, np.uint8)
    mult = C.c_double(0.0)
    cnt = C.c_int64(0)
    rc = L.orc_goss_select_multiclass(_ptr(pr), _ptr(y), n, K, _ptr(w) if w is not None else None, top_rate,
                                      other_rate, seed, round_index, _ptr(rows), _ptr(other),
                                      C.byref(mult), C.byref(cnt))
    assert rc == 0, rc
    return rows[:cnt.value], other, mult.value


def query_starts(counts):
    """Query boundaries (int64, n_queries + 1) from per-query row counts."""
    return np.concatenate([[0], np.cumsum(np.asarray(counts, np.int64))]).astype(np.int64)


def lambdarank(scores, labels, counts, truncation=30, sigma=1.0, norm=True):
    """LambdaRank gradients and hessians of every query, binary64."""
    sc = np.ascontiguousarray(scores, np.float64)
    lab = np.ascontiguousarray(labels, np.float64)
    st = query_starts(counts)
    g = np.zeros(len(sc))
    h = np.zeros(len(sc))
    rc = lib().orc_lambdarank(_ptr(sc), _ptr(lab), _ptr(st), len(st) - 1, truncation, sigma,
                              1 if norm else 0, _ptr(g), _ptr(h))
    if rc != 0:
        raise ValueError("invalid lambdarank input")
    return g, h


def rank_params(counts, **kw):
    """default_params for objective lambdarank over the given query counts;
    the returned starts array must outlive the params."""
    st = query_starts(counts)
    p = default_params(objective=OBJ_LAMBDARANK, **kw)
    p.query_starts = st.ctypes.data
    p.n_queries = len(st) - 1
    return p, st


def categorical_params(n_categories, **kw):
    """default_params with feature f categorical when n_categories[f] > 0;
    the returned array must outlive the params."""
    nc = np.ascontiguousarray(n_categories, np.int32)
    p = default_params(**kw)
    p.n_categories = nc.ctypes.data
    return p, nc


def weighted_params(weights, **kw):
    """default_params with per-row sample weights; the returned array must
    outlive the params."""
    w = np.ascontiguousarray(weights, np.float64)
    p = default_params(**kw)
    p.weights = w.ctypes.data
    return p, w


def cat_split(gh, count, n_categories, total_g=None, total_h=None, total_c=None, lambda_l2=1.0,
              lambda_l1=0.0, min_child_hess=1e-3, min_data_in_leaf=20, max_cat_to_onehot=4,
              max_cat_threshold=32, cat_smooth=10.0, cat_l2=10.0, min_data_per_group=100,
              one_hot_max_size=-1):
    """categorical.find_best_categorical_split on one feature's Float64 plane:
    (found, gain, sorted list of the bins routed left)."""
    gh = np.ascontiguousarray(gh, np.float64).reshape(-1)
    count = np.ascontiguousarray(count, np.int64)
    if total_g is None:
        total_g = float(gh[0::2].sum())
    if total_h is None:
        total_h = float(gh[1::2].sum())
    if total_c is None:
        total_c = int(count.sum())
    g = C.c_double()
    bits = np.zeros(4, np.uint64)
    found = lib().orc_cat_split(_ptr(gh), _ptr(count), n_categories, total_g, total_h, total_c,
                                lambda_l2, lambda_l1, min_child_hess, min_data_in_leaf,
                                max_cat_to_onehot, max_cat_threshold, cat_smooth, cat_l2,
                                min_data_per_group, one_hot_max_size, C.byref(g), _ptr(bits))
    left = [b for b in range(256) if (int(bits[b >> 6]) >> (b & 63)) & 1]
    return bool(found), g.value, left
