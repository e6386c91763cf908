"""Device-level API: a binned matrix resident in HBM and the trainer on it.

Thin Python over include/mojoboost_hip.h (ctypes). Used by the benchmark and
the parity tests, which keep inputs resident between calls.
"""
import ctypes as C

import numpy as np

from . import _lib
from ._lib import check, lib, ptr


def device_count() -> int:
    return int(lib().mbh_device_count())


def bin_dense(x_cm, n_rows, n_features, max_bins=255, min_data_in_bin=3, use_missing=True,
              sample_cnt=200_000, seed=1, categorical=None):
    """Quantile-bin a column-major float64 matrix on the host (the library's
    binning, not the oracle's). Returns (bins_cm uint8, missing_bin int32), or
    with `categorical` (column indices fitted as category tables)
    (bins_cm, missing_bin, n_categories int32)."""
    x_cm = np.ascontiguousarray(x_cm, np.float64).ravel()
    bins = np.zeros(n_rows * n_features, np.uint8)
    mb = np.zeros(n_features, np.int32)
    err = C.create_string_buffer(512)
    if categorical is not None:
        cats = np.ascontiguousarray(categorical, np.int32)
        nc = np.zeros(n_features, np.int32)
        check(lib().mbh_bin_dense_cat(ptr(x_cm), n_rows, n_features, max_bins, min_data_in_bin,
                                      1 if use_missing else 0, sample_cnt, seed, ptr(cats), len(cats),
                                      ptr(bins), ptr(mb), ptr(nc), err, 512), err)
        return bins, mb, nc
    check(lib().mbh_bin_dense(ptr(x_cm), n_rows, n_features, max_bins, min_data_in_bin,
                              1 if use_missing else 0, sample_cnt, seed, ptr(bins), ptr(mb),
                              err, 512), err)
    return bins, mb


def bin_dense_device(x_cm, n_rows, n_features, max_bins=255, min_data_in_bin=3, use_missing=True,
                     sample_cnt=200_000, seed=1, categorical=None):
    """bin_dense with the per-value transform on the GPU (the fit stays on
    the host). Returns (bins_cm uint8, missing_bin int32, n_categories int32,
    times) with times = {fit_ms (host), h2d_ms, transform_ms (the kernel),
    d2h_ms}."""
    x_cm = np.ascontiguousarray(x_cm, np.float64).ravel()
    bins = np.zeros(n_rows * n_features, np.uint8)
    mb = np.zeros(n_features, np.int32)
    nc = np.zeros(n_features, np.int32)
    cats = np.ascontiguousarray(categorical if categorical is not None else [], np.int32)
    t = np.zeros(4, np.float64)
    err = C.create_string_buffer(512)
    check(lib().mbh_bin_dense_device(ptr(x_cm), n_rows, n_features, max_bins, min_data_in_bin,
                                     1 if use_missing else 0, sample_cnt, seed,
                                     ptr(cats) if len(cats) else None, len(cats), ptr(bins), ptr(mb),
                                     ptr(nc), ptr(t), err, 512), err)
    times = dict(fit_ms=float(t[0]), h2d_ms=float(t[1]), transform_ms=float(t[2]), d2h_ms=float(t[3]))
    return bins, mb, nc, times


class Dataset:
    """A column-major uint8 binned matrix and its labels, uploaded once."""

    def __init__(self, bins_cm, n_rows, n_features, n_bins, labels, missing_bin=None,
                 n_categories=None, weights=None):
        L = lib()
        self.n_rows, self.n_features, self.n_bins = int(n_rows), int(n_features), int(n_bins)
        bins_cm = np.ascontiguousarray(bins_cm, dtype=np.uint8).ravel()
        labels = np.ascontiguousarray(labels, dtype=np.float64)
        if bins_cm.size != self.n_rows * self.n_features or labels.size != self.n_rows:
            raise ValueError("bins must be n_rows * n_features and labels n_rows")
        mb = None if missing_bin is None else np.ascontiguousarray(missing_bin, np.int32)
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        check(L.mbh_dataset_create(ptr(bins_cm), self.n_rows, self.n_features, self.n_bins,
                                   ptr(mb), ptr(labels), C.byref(h), err, 1024), err)
        self.h = h
        if n_categories is not None:
            self.set_categorical(n_categories)
        if weights is not None:
            self.set_weights(weights)

    def set_categorical(self, n_categories):
        """n_categories[f] > 0 marks feature f categorical (bins 1..n, bin 0
        missing/unseen)."""
        nc = np.ascontiguousarray(n_categories, np.int32)
        err = C.create_string_buffer(512)
        check(lib().mbh_dataset_set_categorical(self.h, ptr(nc), err, 512), err)

    def free(self):
        if getattr(self, "h", None):
            lib().mbh_dataset_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def set_weights(self, weights):
        """Per-row sample weights for later trainings (None clears them)."""
        err = C.create_string_buffer(512)
        if weights is None:
            check(lib().mbh_dataset_set_weights(self.h, None, 0, err, 512), err)
            return
        w = np.ascontiguousarray(weights, np.float64)
        check(lib().mbh_dataset_set_weights(self.h, ptr(w), w.size, err, 512), err)

    def set_groups(self, counts):
        """Query groups for objective lambdarank: rows per query, in row order."""
        c = np.ascontiguousarray(counts, np.int32)
        err = C.create_string_buffer(512)
        check(lib().mbh_dataset_set_groups(self.h, ptr(c), len(c), err, 512), err)

    def lambdarank(self, raw, **params):
        """LambdaRank gradients and hessians (binary64) of raw scores."""
        p = _lib.mbh_params(**params)
        raw = np.ascontiguousarray(raw, np.float64)
        g = np.zeros(self.n_rows)
        h = np.zeros(self.n_rows)
        err = C.create_string_buffer(1024)
        check(lib().mbh_lambdarank(self.h, C.byref(p), ptr(raw), ptr(g), ptr(h), err, 1024), err)
        return g, h

    def train(self, **params):
        p = _lib.mbh_params(**params)
        f = C.c_void_p()
        err = C.create_string_buffer(1024)
        check(lib().mbh_train(self.h, C.byref(p), C.byref(f), err, 1024), err)
        return Fit(f, self.n_rows, p.learning_rate)

    def objective_quantize(self, raw, round_index=0, **params):
        n = self.n_rows
        p = _lib.mbh_params(**params)
        g = np.zeros(n, np.float32)
        h = np.zeros(n, np.float32)
        qg = np.zeros(n, np.int8)
        qh = np.zeros(n, np.int8)
        sc = np.zeros(2)
        err = C.create_string_buffer(1024)
        raw = np.ascontiguousarray(raw, np.float64)
        check(lib().mbh_objective_quantize(self.h, C.byref(p), ptr(raw), round_index, ptr(g),
                                           ptr(h), ptr(qg), ptr(qh), ptr(sc), err, 1024), err)
        return g, h, qg, qh, sc

    def objective_quantize32(self, raw, round_index=0, **params):
        """Either lattice with int32 values: (grad, hess, q_grad, q_hess,
        [grad units, hess units, sum|g|, sum|h|, int16 misfits of grad,
        of hess]) -- the sums are the device magnitude reduction's under
        quant_scale_rule=1, the misfit counts the int16 staging's
        (quant_staging=1), else 0."""
        n = self.n_rows
        p = _lib.mbh_params(**params)
        g = np.zeros(n, np.float32)
        h = np.zeros(n, np.float32)
        qg = np.zeros(n, np.int32)
        qh = np.zeros(n, np.int32)
        sc = np.zeros(6)
        err = C.create_string_buffer(1024)
        raw = np.ascontiguousarray(raw, np.float64)
        check(lib().mbh_objective_quantize32(self.h, C.byref(p), ptr(raw), round_index, ptr(g),
                                             ptr(h), ptr(qg), ptr(qh), ptr(sc), err, 1024), err)
        return g, h, qg, qh, sc

    def histogram32(self, q_grad, q_hess, rows=None):
        """Histogram of int32 quantized values (the magnitude-sum lattice)."""
        out = np.zeros(self.n_features * self.n_bins * 3, np.int32)
        r = None if rows is None else np.ascontiguousarray(rows, np.int32)
        err = C.create_string_buffer(1024)
        check(lib().mbh_histogram32(self.h, ptr(np.ascontiguousarray(q_grad, np.int32)),
                                    ptr(np.ascontiguousarray(q_hess, np.int32)), ptr(r),
                                    0 if r is None else len(r), ptr(out), err, 1024), err)
        return out.reshape(self.n_features, self.n_bins, 3)

    def histogram(self, q_grad, q_hess, rows=None, quant_bins=4):
        out = np.zeros(self.n_features * self.n_bins * 3, np.int32)
        r = None if rows is None else np.ascontiguousarray(rows, np.int32)
        err = C.create_string_buffer(1024)
        check(lib().mbh_histogram(self.h, ptr(np.ascontiguousarray(q_grad, np.int8)),
                                  ptr(np.ascontiguousarray(q_hess, np.int8)), ptr(r),
                                  0 if r is None else len(r), quant_bins, ptr(out), err, 1024), err)
        return out.reshape(self.n_features, self.n_bins, 3)

    def histogram_fp32(self, grad, hess, rows=None):
        """fp64 sums of fp32 grad/hess per (feature, bin), and counts."""
        cells = self.n_features * self.n_bins
        gh = np.zeros(2 * cells)
        cnt = np.zeros(cells, np.int64)
        g = np.ascontiguousarray(grad, np.float32)
        h = np.ascontiguousarray(hess, np.float32)
        r = None if rows is None else np.ascontiguousarray(rows, np.int32)
        err = C.create_string_buffer(1024)
        check(lib().mbh_histogram_fp32(self.h, ptr(g), ptr(h), ptr(r), 0 if r is None else len(r),
                                       ptr(gh), ptr(cnt), err, 1024), err)
        return gh, cnt

    def bench_root_histogram(self, reps=20):
        """(mean, min) histogram-kernel ms and mean histogram + merge ms of a
        root build over all rows."""
        out = np.zeros(3)
        err = C.create_string_buffer(1024)
        check(lib().mbh_bench_root_histogram(self.h, reps, ptr(out), err, 1024), err)
        return float(out[0]), float(out[1]), float(out[2])


class Fit:
    """Trees grown by mbh_train, as flat arrays."""

    def __init__(self, handle, n_rows, learning_rate=0.1):
        L = lib()
        self.h = handle
        self.n_rows = n_rows
        self.learning_rate = float(learning_rate)
        self.n_trees = int(L.mbh_fit_num_trees(handle))
        self.num_class = int(L.mbh_fit_num_class(handle))
        nn = int(L.mbh_fit_total_nodes(handle))
        self.base = np.zeros(self.num_class)
        self.off = np.zeros(self.n_trees + 1, np.int64)
        i32 = lambda: np.zeros(nn, np.int32)
        f64 = lambda: np.zeros(nn, np.float64)
        self.feature, self.threshold, self.left, self.right = i32(), i32(), i32(), i32()
        self.value, self.default_left, self.missing_bin = f64(), i32(), i32()
        self.gain, self.count = f64(), f64()
        L.mbh_fit_arrays(handle, ptr(self.base), ptr(self.off), ptr(self.feature),
                         ptr(self.threshold), ptr(self.left), ptr(self.right), ptr(self.value),
                         ptr(self.default_left), ptr(self.missing_bin), ptr(self.gain),
                         ptr(self.count))
        self.cat_bits = np.zeros((nn, 4), np.uint64)
        L.mbh_fit_cat_bits(handle, ptr(self.cat_bits))
        names = ("train_seconds", "hist_ms", "hist_bytes", "hist_rows_features",
                 "hist_builds", "root_bytes", "root_ms", "trees_grown", "growth_ms",
                 "root_growth_ms", "iterations", "expansions", "rows_built", "rows_parted",
                 "expand_launches", "expand_ms", "expand_bytes", "partition_ms", "accum_ms",
                 "accum_bytes", "root_quantizer_bytes",
                 "partition_bytes")
        st = np.zeros(len(names))
        count = L.mbh_fit_stats(handle, ptr(st), len(names))
        assert count == len(names), count
        self.stats = dict(zip(names, (float(v) for v in st)))
        # time_histograms fits: one row per expansion launch (tree,
        # iteration, rows partitioned, rows accumulated, partition ms,
        # accumulation ms); empty otherwise
        n_log = int(L.mbh_fit_launch_log(handle, None, 0))
        log = np.zeros(n_log)
        if n_log:
            L.mbh_fit_launch_log(handle, ptr(log), n_log)
        self.launch_log = log.reshape(-1, 6)

    def tree(self, t):
        a, b = self.off[t], self.off[t + 1]
        return {k: getattr(self, k)[a:b] for k in
                ("feature", "threshold", "left", "right", "value", "default_left",
                 "missing_bin", "gain", "count")}

    def predict_binned(self, bins_cm, n_rows, n_features, tree_begin=0, tree_end=None):
        """Raw scores of trees [tree_begin, tree_end) on the device, from
        column-major uint8 bins; the base score is added when the range
        starts at tree 0."""
        tree_end = self.n_trees if tree_end is None else tree_end
        bins_cm = np.ascontiguousarray(bins_cm, np.uint8).ravel()
        out = np.zeros(n_rows * self.num_class)
        err = C.create_string_buffer(512)
        check(lib().mbh_predict_binned(
            ptr(bins_cm), n_rows, n_features, self.num_class, self.learning_rate,
            ptr(self.base) if tree_begin == 0 else None, ptr(self.off), tree_begin, tree_end,
            ptr(self.feature), ptr(self.threshold), ptr(self.left), ptr(self.right),
            ptr(self.value), ptr(self.default_left), ptr(self.missing_bin),
            ptr(self.cat_bits) if self.cat_bits.any() else None, ptr(out), err, 512), err)
        return out

    def train_raw(self):
        out = np.zeros(self.n_rows * self.num_class)
        err = C.create_string_buffer(256)
        check(lib().mbh_fit_train_raw(self.h, ptr(out), err, 256), err)
        return out

    def __del__(self):
        try:
            if getattr(self, "h", None):
                lib().mbh_fit_free(self.h)
                self.h = None
        except Exception:
            pass


def exp_sigmoid(x):
    x = np.ascontiguousarray(x, np.float64)
    e = np.zeros_like(x)
    s = np.zeros_like(x)
    err = C.create_string_buffer(512)
    check(lib().mbh_exp_sigmoid(ptr(x), x.size, ptr(e), ptr(s), err, 512), err)
    return e, s
