"""Writes tests/golden/full_size_digests.json: the CPU oracle's fits of
BASELINE.json's C2, C4 and C5 workloads at their full sizes (the bench's
seeded data, binned by the library's host binning), as per-tree digests.

    python tests/golden/make_full_size_digests.py [c2|c4|c5 ...]

C2 is the north star's target, all 500 trees (about 20 minutes on 8 cores);
C4 and C5 take their first trees or rounds. The GPU tests in
tests/test_gpu_full_size.py train the same workloads on the device and
compare digests tree by tree. Only the named workloads are rewritten.
"""
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

import full_size as FS  # noqa: E402
import oracle_lib as O  # noqa: E402

# trees (rounds for C5) compared at full size
ITERATIONS = {"c2": 500, "c4": 12, "c5": 8}


def make(name):
    t0 = time.perf_counter()
    bins, missing, ncat, y, n, F, nb = FS.data(name)
    t_data = time.perf_counter() - t0
    kw = FS.params(name, ITERATIONS[name])
    threads = os.cpu_count() or 1
    p = O.default_params(num_grad_quant_bins=4, n_threads=threads, **kw)
    if ncat is not None:
        p.n_categories = ncat.ctypes.data  # ncat outlives the oracle call
    t1 = time.perf_counter()
    ref = O.train(bins, n, F, nb, y, p, missing_bin=missing)
    t_train = time.perf_counter() - t1
    raw = ref.train_raw(n)
    entry = {
        "params": kw,
        "rows": n,
        "features": F,
        "max_bin": nb,
        "bins_sha256": FS.sha(bins, np.asarray(missing, np.int32)),
        "labels_sha256": FS.sha(np.asarray(y, np.float64)),
        "n_categories": None if ncat is None else [int(v) for v in ncat],
        "n_trees": int(ref.n_trees),
        "base_bits": [f"{int(v):016x}" for v in np.asarray(ref.base, np.float64).view(np.uint64)],
        "trees": FS.tree_digests(ref),
        "train_raw_sha256": FS.sha(raw.view(np.uint64)),
        "oracle_threads": threads,
        "oracle_seconds": round(t_train, 1),
    }
    print(f"{name}: data {t_data:.1f}s, oracle {ref.n_trees} trees in {t_train:.1f}s", flush=True)
    return entry


def main(names):
    out = json.loads(FS.DIGESTS.read_text()) if FS.DIGESTS.exists() else {}
    for name in names:
        out[name] = make(name)
        FS.DIGESTS.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:] or ["c4", "c5", "c2"])
