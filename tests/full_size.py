"""Full-size parity at BASELINE.json's own shapes: the workloads' data (the
bench's seeded generators), binned by the library's host binning, and per-tree
digests of a fit (structure plus the binary64 bits of every node's value,
gain and count), so a 500-tree oracle run made once on the CPU can be
compared with a GPU run without shipping the trees.

The digests of the oracle's fits are the data fixture
tests/golden/full_size_digests.json, written by
tests/golden/make_full_size_digests.py.
"""
import hashlib
import json
from pathlib import Path

import numpy as np

from bench import WORKLOADS, workload_data

DIGESTS = Path(__file__).resolve().parent / "golden" / "full_size_digests.json"

# the bench's training parameters (bench.py main), per workload
COMMON = dict(min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.1)


def params(name, num_iterations):
    wl = WORKLOADS[name]
    return dict(num_leaves=wl["leaves"], num_iterations=num_iterations, **COMMON, **wl["params"])


def data(name):
    """(bins, missing, n_categories or None, labels, n_rows, F, max_bin) of a
    workload at its full size, binned as the bench bins it."""
    from mojoboost_amd import device

    wl = WORKLOADS[name]
    n, F, nb = wl["rows"], wl["features"], wl["max_bin"]
    x, y = workload_data(name, n)
    cats = wl.get("categorical")
    if cats:
        bins, missing, ncat = device.bin_dense(x.ravel(), n, F, max_bins=nb, categorical=cats)
    else:
        (bins, missing), ncat = device.bin_dense(x.ravel(), n, F, max_bins=nb), None
    del x
    return bins, missing, ncat, y, n, F, nb


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tree_digests(fit):
    """One 64-bit digest per tree: feature, threshold, children, default
    direction, missing bin, category sets, and the bits of value, gain and
    count. `fit` is an oracle Model or a device Fit (the same flat arrays)."""
    out = []
    for t in range(fit.n_trees):
        a, b = int(fit.off[t]), int(fit.off[t + 1])
        parts = [np.asarray(getattr(fit, k)[a:b], np.int32)
                 for k in ("feature", "threshold", "left", "right", "default_left", "missing_bin")]
        parts.append(np.asarray(fit.cat_bits[a:b], np.uint64))
        parts += [np.asarray(getattr(fit, k)[a:b], np.float64).view(np.uint64)
                  for k in ("value", "gain", "count")]
        out.append(sha(*parts)[:16])
    return out


def load():
    return json.loads(DIGESTS.read_text())
