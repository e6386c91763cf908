"""Benchmark: GBDT training on one MI355X, BASELINE.json configs[1] (C2) by
default; --workload c3|c4|c5 measures configs[2..4] the same way.

Workload: 10.5M rows x 28 features (21 N(0,1), 7 products/abs of pairs),
binary label ~ Bernoulli(sigmoid(sum of 8 random pairwise terms)), logistic
objective, max_bin 255, num_leaves 255, quantized gradients (int8 g/h,
int32 histogram cells). Synthetic and seeded; generated here.

A "step" is one boosting iteration (one tree; one round of K trees for
multiclass). The timed region trains --steps trees from scratch on the
HBM-resident dataset, bracketed by device synchronization (the library syncs
before returning): `ms_per_step`. Whatever --steps says, every run also
trains the workload's full tree count (500 for C2) from scratch and times it:
`train_sec_per_<full>_trees` is that measured time, never an extrapolation.

`value` is the histogram-build throughput of an instrumented run of the full
training: the algorithmic bytes of every histogram the run accumulated -- the
root and each expansion's smaller child, speculative expansions included --
m rows * (F + gh) (uint8 bins + the g/h pair: 2 bytes int8, 8 bytes fp32; row
ids, LDS traffic and partial writes not counted), over the durations of the
kernels that accumulate them (k_hist for the root, k_accum for the children).
The root build that training runs also quantizes (max-abs lattice): the
quantizer's own bytes (binary32 g, h in, the int8 pair out) are reported
apart (`root_quantizer_bytes_per_tree`), never in `value`.
The durations come from HIP events that the runtime records at each kernel's
own start and end (hipExtLaunchKernel), on the stream the kernel runs on, so
they are the kernel times rocprofv3's kernel trace reports. `roofline` prices
k_accum alone; `traffic` is its HBM bytes per launch from rocprofv3 PMC
counters. The conservative figure that charges every growth kernel
(partition, accumulation, partial merge and scan, planning) against the
committed trees' builds only is reported as `hist_gbs_committed_over_growth`.

records_layout: the same full training with leaves holding their rows as
whole records (partition_mode=1: the partition moves records, the histogram
streams them) instead of row ids (the default, which gathers each record by
id), timed and instrumented the same way, its trees checked identical.

cpu_baseline: the CPU oracle (a C++ restatement of the reference's CPU
trainer; the reference itself is Mojo and cannot run here) on the first
--cpu-trees trees of the same workload on all rows (a bounded sample of
10-20 s), whose trees are also compared bit for bit with the GPU's, on the
host cores this process may use, at most 16 (a GPU box's CPU share for one
GPU); the CPU model is reported beside it.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "hist-build GB/s (% HBM peak) + train sec/500 trees, 10.5M×28 logistic, 1 GPU"
# the same metric on the other BASELINE configurations
METRICS = {
    "c2": METRIC,
    "c3": "hist-build GB/s (% HBM peak) + train sec/500 trees, 10.5M×28 logistic, fp32 g/h + GOSS, 1 GPU",
    "c4": "hist-build GB/s (% HBM peak) + train sec/200 trees, 400k×2000 logistic, 63 bins, 1 GPU",
    "c5": "hist-build GB/s (% HBM peak) + train sec/100 rounds, 2M×50 softmax 10 classes, 1 GPU",
}


def c2_data(n_rows, seed=0x5EED0002):
    """C2 features (float32 values held in a column-major float64 matrix) and
    labels. The intercept puts the positive rate near 53%."""
    rng = np.random.default_rng(seed)
    x = np.empty((28, n_rows), np.float64)
    for f in range(21):
        x[f] = rng.standard_normal(n_rows, dtype=np.float32)
    pairs = [(0, 1), (2, 3), (4, 5), (6, 7), (8, 9), (10, 11), (12, 13)]
    for i, (a, b) in enumerate(pairs):
        prod = (x[a] * x[b]).astype(np.float32)
        x[21 + i] = prod if i % 2 == 0 else np.abs(prod)
    terms = rng.integers(0, 21, size=(8, 2))
    w = rng.uniform(-1.0, 1.0, size=8)
    logit = np.zeros(n_rows)
    for i, (a, b) in enumerate(terms):
        logit += w[i] * x[a] * x[b]
    # intercept solving mean(sigmoid(c + logit)) = 0.53 (Newton on a fixed
    # 200k-row prefix, so it is a deterministic function of the seed)
    c, s = 0.0, logit[:200_000]
    for _ in range(20):
        p = 1.0 / (1.0 + np.exp(-(c + s)))
        c -= (p.mean() - 0.53) / max(1e-12, (p * (1.0 - p)).mean())
    logit += c
    y = (rng.uniform(size=n_rows) < 1.0 / (1.0 + np.exp(-logit))).astype(np.float64)
    return x, y


def c4_data(n_rows, n_features=2000, seed=0x5EED0004):
    """C4: N(0,1) features, label = sign of a sparse 50-feature linear model
    plus noise."""
    rng = np.random.default_rng(seed)
    x = np.empty((n_features, n_rows), np.float64)
    for f in range(n_features):
        x[f] = rng.standard_normal(n_rows, dtype=np.float32)
    idx = rng.choice(n_features, 50, replace=False)
    w = rng.standard_normal(50)
    score = np.zeros(n_rows)
    for i, f in enumerate(idx):
        score += w[i] * x[f]
    y = (score + 0.5 * rng.standard_normal(n_rows) > 0).astype(np.float64)
    return x, y


def c5_data(n_rows, n_classes=10, seed=0x5EED0005):
    """C5: 40 N(0,1) columns and 10 integer columns of cardinality 4-64
    (uniform); the class is the argmax of a random linear score over the
    continuous columns plus a random effect per category value, plus Gumbel
    noise."""
    rng = np.random.default_rng(seed)
    x = np.empty((50, n_rows), np.float64)
    scores = np.zeros((n_classes, n_rows))
    w = rng.standard_normal((n_classes, 40)) * 0.5
    for f in range(40):
        x[f] = rng.standard_normal(n_rows, dtype=np.float32)
        scores += np.outer(w[:, f], x[f])
    cards = rng.integers(4, 65, size=10)
    for j in range(10):
        c = rng.integers(0, cards[j], size=n_rows)
        x[40 + j] = c
        effect = rng.standard_normal((n_classes, cards[j])) * 0.5
        scores += effect[:, c]
    scores += rng.gumbel(size=(n_classes, n_rows))
    y = np.argmax(scores, axis=0).astype(np.float64)
    return x, y


# BASELINE.json configs[1..4]; the driver's default line is C2 (the metric's
# configuration), the others are measured the same way when named.
WORKLOADS = {
    "c2": dict(rows=10_500_000, features=28, max_bin=255, leaves=255, trees=500, classes=1,
               gh_bytes=2, params=dict(objective=1, use_quantized_grad=1),
               cpu_sample=16, desc="C2: 10.5M x 28 binary logistic, max_bin 255, num_leaves 255, "
                    "quantized gradients (int8 g/h, int32 histogram bins)",
               dtype="int8 g/h, int32 cells"),
    "c3": dict(rows=10_500_000, features=28, max_bin=255, leaves=255, trees=500, classes=1,
               gh_bytes=8, params=dict(objective=1, use_quantized_grad=0, goss=1, top_rate=0.2,
                                       other_rate=0.1),
               cpu_sample=14, desc="C3: the C2 workload with fp32 gradients (fp64 histogram sums) and GOSS "
                    "(top_rate 0.2, other_rate 0.1, warmup 10 rounds)",
               dtype="fp32 g/h, fp64 sums"),
    "c4": dict(rows=400_000, features=2000, max_bin=63, leaves=127, trees=200, classes=1,
               gh_bytes=2, params=dict(objective=1, use_quantized_grad=1),
               cpu_sample=10, desc="C4: 400k x 2000 binary logistic (sparse linear label), max_bin 63, "
                    "num_leaves 127, quantized gradients; 16 feature tiles",
               dtype="int8 g/h, int32 cells"),
    "c5": dict(rows=2_000_000, features=50, max_bin=255, leaves=63, trees=100, classes=10,
               gh_bytes=2, params=dict(objective=2, num_class=10, use_quantized_grad=1),
               cpu_sample=6, categorical=list(range(40, 50)),
               desc="C5: 2M x 50 (40 continuous, 10 integer columns of cardinality 4-64 split as "
                    "category sets) softmax, 10 classes, max_bin 255, num_leaves 63, quantized "
                    "gradients per class; a step is one round of 10 trees",
               dtype="int8 g/h, int32 cells"),
}


def workload_data(name, n_rows):
    if name in ("c2", "c3"):
        return c2_data(n_rows)
    if name == "c4":
        return c4_data(n_rows)
    return c5_data(n_rows)


def cpu_model():
    """The host CPU's model name with its family / model / stepping numbers
    and clock (/proc/cpuinfo; a virtualized host may report only the
    vendor's product line as the name), or None."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (t.strip() for t in line.split(":", 1))
                if k in ("model name", "cpu family", "model", "stepping", "cpu MHz") and k not in fields:
                    fields[k] = v
            elif fields:
                break
    except OSError:
        return None
    if "model name" not in fields:
        return None
    extra = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping", "cpu MHz") if k in fields)
    return f"{fields['model name']} ({extra})" if extra else fields["model name"]


def host_cores():
    """(cores used, cores visible): the CPUs this process may run on, at most
    16, a GPU box's CPU share for one GPU."""
    try:
        visible = len(os.sched_getaffinity(0))
    except AttributeError:
        visible = os.cpu_count() or 1
    return min(16, visible), visible


def traffic_per_launch(workload):
    """HBM bytes per k_accum launch measured by rocprofv3 (FETCH_SIZE and
    WRITE_SIZE passes over the same workload, calibrated against a plain
    device copy), as committed under profiles/; None when absent."""
    p = ROOT / "profiles" / f"k_accum_{workload}_traffic.json"
    if not p.exists():
        return None
    return json.loads(p.read_text()).get("traffic_bytes_per_launch")


def rocprof_summary(path):
    """Markdown table of a rocprofv3 CSV: per-kernel durations from a
    *_kernel_stats.csv, or per-kernel mean counter values per dispatch from a
    *_counter_collection.csv."""
    import csv
    import collections
    rows = list(csv.DictReader(open(path)))
    if rows and "AverageNs" in rows[0]:
        print("| kernel | calls | total ms | avg us | min us | max us | % |")
        print("|---|---:|---:|---:|---:|---:|---:|")
        for r in rows:
            print(f"| `{r['Name'][:60]}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.2f} | "
                  f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                  f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
        return 0
    agg = collections.defaultdict(lambda: [0, 0.0])
    for r in rows:
        key = (r.get("Kernel_Name", "")[:60], r.get("Counter_Name", ""))
        agg[key][0] += 1
        agg[key][1] += float(r.get("Counter_Value", 0) or 0)
    print("| kernel | counter | dispatches | mean per dispatch |")
    print("|---|---|---:|---:|")
    for (k, c), (n, sm) in sorted(agg.items(), key=lambda x: -x[1][1]):
        print(f"| `{k}` | {c} | {n} | {sm / n:.1f} |")
    return 0


SIZE_EDGES = [1, 16_384, 65_536, 262_144, 1_048_576, 4_194_304]


def size_classes(log, rows_col, ms_col, bytes_per_row):
    """Launches of one expansion kernel by rows per launch: count, rows,
    mean duration, share of the kernel's time and algorithmic GB/s per
    class. `log` is a fit's launch_log (tree, iteration, rows partitioned,
    rows accumulated, partition ms, accumulation ms)."""
    rows, ms = log[:, rows_col], log[:, ms_col]
    total = max(1e-12, float(ms.sum()))
    edges = [0] + SIZE_EDGES + [float("inf")]
    out = []
    for lo, hi in zip(edges[:-1], edges[1:]):
        sel = (rows >= lo) & (rows < hi) if lo > 0 else rows == 0
        if not sel.any():
            continue
        r, t = float(rows[sel].sum()), float(ms[sel].sum())
        out.append({"rows": "0" if lo == 0 else f"{int(lo)}-{'' if hi == float('inf') else int(hi)}",
                    "launches": int(sel.sum()), "rows_per_launch": round(r / sel.sum(), 1),
                    "avg_us": round(t / sel.sum() * 1e3, 2), "time_share": round(t / total, 4),
                    "gbs": round(r * bytes_per_row / (t * 1e-3) / 1e9, 1) if t > 0 else None})
    return out


def size_table_md(title, classes):
    lines = [f"### {title}", "", "| rows per launch | launches | avg rows | avg us | share of time | GB/s |",
             "|---|---:|---:|---:|---:|---:|"]
    for c in classes:
        lines.append(f"| {c['rows']} | {c['launches']} | {c['rows_per_launch']:.0f} | {c['avg_us']:.2f} | "
                     f"{c['time_share']:.1%} | {c['gbs'] if c['gbs'] is not None else '-'} |")
    return "\n".join(lines) + "\n"


def copy_probe(mib):
    """One hipMemcpy device-to-device of `mib` MiB: the runtime's blit kernel
    reads and writes exactly that many bytes, which calibrates the HBM byte
    counters (FETCH_SIZE, WRITE_SIZE) the histogram kernels are read with."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    n = mib << 20
    a, b = C.c_void_p(), C.c_void_p()
    for p in (a, b):
        if hip.hipMalloc(C.byref(p), C.c_size_t(n)) != 0:
            print(json.dumps({"error": "hipMalloc failed"}))
            return 1
    hip.hipMemset(a, 1, C.c_size_t(n))
    rc = hip.hipMemcpy(b, a, C.c_size_t(n), 3)  # hipMemcpyDeviceToDevice
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)
    print(json.dumps({"copy_probe_mib": mib, "rc": rc}))
    return 0 if rc == 0 else 1


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--steps", type=int, default=None,
                    help="trees (rounds for c5); default: the workload's full count")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--rows", type=int, default=None)
    ap.add_argument("--cpu-trees", type=int, default=None,
                    help="oracle sample: trees (rounds for c5); default per workload")
    ap.add_argument("--no-instrumented", action="store_true")
    ap.add_argument("--launch-table", default=None,
                    help="also write the expansion kernels' size-class tables (markdown) to this file")
    ap.add_argument("--partition-mode", type=int, default=0,
                    help="leaf rows as 0 automatic, 1 records, 2 row ids (mbh_params.partition_mode)")
    ap.add_argument("--rocprof-summary", default=None,
                    help="only summarize a rocprofv3 CSV (kernel_stats or counter_collection) "
                         "as a markdown table")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run one device-to-device copy of this many MiB (the "
                         "calibration kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU row sharding is a "
                          "design only (rows sharded per GPU, histograms all-reduced), "
                          "--gpus must be 1"}))
        return 2

    if args.rocprof_summary:
        return rocprof_summary(args.rocprof_summary)
    if args.copy_probe_mib > 0:
        return copy_probe(args.copy_probe_mib)

    from mojoboost_amd import device

    if device.device_count() < 1:
        print(json.dumps({"error": "no gfx950 GPU visible"}))
        return 1
    wl = WORKLOADS[args.workload]
    F, NB, L, K = wl["features"], wl["max_bin"], wl["leaves"], wl["classes"]
    GH = wl["gh_bytes"]
    if args.rows is None:
        args.rows = wl["rows"]
    if args.steps is None:
        args.steps = wl["trees"]
    if args.cpu_trees is None:
        args.cpu_trees = wl["cpu_sample"]
    t0 = time.perf_counter()
    x, y = workload_data(args.workload, args.rows)
    cats = wl.get("categorical")
    n_cat = None
    # binning, reported apart from training: the host path (fit + transform
    # on the host's threads) and the device path (the same fit on the host,
    # the per-value transform as one kernel); both must give the same bytes
    tb = time.perf_counter()
    if cats:
        bins, missing, n_cat = device.bin_dense(x.ravel(), args.rows, F, max_bins=NB, categorical=cats)
    else:
        bins, missing = device.bin_dense(x.ravel(), args.rows, F, max_bins=NB)
    host_bin_s = time.perf_counter() - tb
    tb = time.perf_counter()
    dbins, dmissing, dn_cat, btimes = device.bin_dense_device(x.ravel(), args.rows, F, max_bins=NB,
                                                              categorical=cats)
    dev_bin_s = time.perf_counter() - tb
    cells = args.rows * F
    binning = {
        "host_fit_and_transform_s": round(host_bin_s, 4),
        "device_path_s": round(dev_bin_s, 4),
        "device_fit_ms_host": round(btimes["fit_ms"], 2),
        "device_h2d_ms": round(btimes["h2d_ms"], 2),
        "device_transform_kernel_ms": round(btimes["transform_ms"], 4),
        "device_d2h_ms": round(btimes["d2h_ms"], 2),
        "transform_kernel_gbs": round(cells * 9 / (btimes["transform_ms"] * 1e-3) / 1e9, 1),
        "transform_bytes_per_value": 9,
        "bins_identical": bool(np.array_equal(bins, dbins) and np.array_equal(missing, dmissing)),
    }
    del x, dbins
    t_data = time.perf_counter() - t0
    print(f"[bench] {args.workload}: data {args.rows}x{F} generated+binned in {t_data:.1f}s, "
          f"label mean {y.mean():.3f}", file=sys.stderr, flush=True)
    ds = device.Dataset(bins, args.rows, F, NB, y, missing_bin=missing, n_categories=n_cat)
    kw = dict(num_leaves=L, min_data_in_leaf=20, lambda_l2=1.0, learning_rate=0.1,
              num_grad_quant_bins=4, stochastic_rounding=1, **wl["params"])
    if args.partition_mode:
        kw["partition_mode"] = args.partition_mode
    if args.warmup > 0:
        ds.train(num_iterations=args.warmup, **kw)
    print("[bench] warmup done", file=sys.stderr, flush=True)

    t1 = time.perf_counter()
    fit = ds.train(num_iterations=args.steps, **kw)
    wall = time.perf_counter() - t1
    trees = fit.n_trees
    print(f"[bench] timed: {args.steps} steps in {wall:.3f}s ({trees} trees kept)",
          file=sys.stderr, flush=True)
    # the workload's full training, measured whatever --steps is
    full = wl["trees"]
    if args.steps == full:
        full_fit, full_wall = fit, wall
    else:
        t2 = time.perf_counter()
        full_fit = ds.train(num_iterations=full, **kw)
        full_wall = time.perf_counter() - t2
    print(f"[bench] full training: {full} steps in {full_wall:.3f}s ({full_fit.n_trees} trees kept)",
          file=sys.stderr, flush=True)

    st = None
    stat_steps = full
    if not args.no_instrumented:
        ifit = ds.train(num_iterations=full, time_histograms=1, **kw)
        st = ifit.stats
        launch_log = ifit.launch_log
        same = np.array_equal(ifit.threshold, full_fit.threshold) and np.array_equal(
            ifit.value.view(np.uint64), full_fit.value.view(np.uint64))
        print(f"[bench] instrumented full run done (trees identical to the timed run: {same})",
              file=sys.stderr, flush=True)
    # the other leaf-row layout, measured the same way (full training, then
    # its instrumented run): leaves holding their rows as whole records
    # (partition_mode=1) stream the histogram, row ids (the default) gather it
    alt = None
    if not args.no_instrumented and not args.partition_mode and wl["params"].get("use_quantized_grad") \
            and F + GH <= 64:
        akw = dict(kw, partition_mode=1)
        t3 = time.perf_counter()
        afit = ds.train(num_iterations=full, **akw)
        alt_wall = time.perf_counter() - t3
        ast = ds.train(num_iterations=full, time_histograms=1, **akw).stats
        same_alt = np.array_equal(afit.threshold, full_fit.threshold) and np.array_equal(
            afit.value.view(np.uint64), full_fit.value.view(np.uint64))
        alt = {"partition_mode": 1, "leaf_rows": "records",
               f"train_sec_per_{full}_{'rounds' if K > 1 else 'trees'}": round(alt_wall, 3),
               "value": round((ast["root_bytes"] + ast["accum_bytes"]) / ((ast["root_ms"] + ast["accum_ms"]) * 1e-3)
                              / 1e9, 2),
               "accum_gbs": round(ast["accum_bytes"] / (ast["accum_ms"] * 1e-3) / 1e9, 1),
               "accum_kernel_avg_ms": round(ast["accum_ms"] / max(1.0, ast["expand_launches"]), 5),
               "partition_ms_per_tree": round(ast["partition_ms"] / full, 4),
               "traffic": traffic_per_launch(args.workload + "rec"),
               "trees_identical_to_row_ids": bool(same_alt)}
        print(f"[bench] records layout: {full} steps in {alt_wall:.3f}s (trees identical: {same_alt})",
              file=sys.stderr, flush=True)
    root_mean_ms, root_min_ms, root_merged_ms = ds.bench_root_histogram(reps=20)

    # CPU baseline on the same bins: the first --cpu-trees trees of the workload.
    cpu = None
    parity = None
    if args.cpu_trees > 0:
        sys.path.insert(0, str(ROOT / "tests"))
        import oracle_lib as O

        cores, visible = host_cores()
        oparams = {k: v for k, v in kw.items()
                   if k not in ("num_grad_quant_bins", "stochastic_rounding", "partition_mode")}
        p = O.default_params(num_iterations=args.cpu_trees, num_grad_quant_bins=4, n_threads=cores,
                             **oparams)
        if n_cat is not None:
            p.n_categories = n_cat.ctypes.data  # n_cat outlives the oracle call
        tc = time.perf_counter()
        ref = O.train(bins, args.rows, F, NB, y, p, missing_bin=missing)
        cpu_s = time.perf_counter() - tc
        k = min(ref.n_trees, full_fit.n_trees)
        a, b = ref.off[k], full_fit.off[k]
        same_shape = bool(a == b and all(
            np.array_equal(getattr(ref, f)[:a], getattr(full_fit, f)[:b])
            for f in ("feature", "threshold", "left", "right", "default_left", "cat_bits")))
        if wl["params"].get("use_quantized_grad"):
            parity = same_shape and bool(np.array_equal(ref.value[:a].view(np.uint64),
                                                        full_fit.value[:b].view(np.uint64)))
            how = "bit-identical"
        else:
            parity = same_shape and bool(np.allclose(ref.value[:a], full_fit.value[:b], rtol=1e-5, atol=0))
            how = "same splits, values within 1e-5"
        per_step = cpu_s / max(1, args.cpu_trees)
        unit_steps = "rounds" if K > 1 else "trees"
        cpu = {"value": round(per_step * full, 2), "unit": f"s/{full} {unit_steps}", "cores": cores,
               "kind": "port", "cpu_model": cpu_model(), "cpus_visible": visible,
               "sample": f"first {args.cpu_trees} {unit_steps} of the {args.workload.upper()} workload "
                         f"on all {args.rows} rows ({cpu_s:.1f}s, {per_step:.2f}s each, "
                         f"scaled x{full / args.cpu_trees:.1f} to {full} {unit_steps}) on {cores} "
                         f"threads; trees {how} to GPU: {parity}"}
        print(f"[bench] cpu oracle {args.cpu_trees} {unit_steps} in {cpu_s:.1f}s", file=sys.stderr,
              flush=True)

    # the root build of stored pairs (k_hist without the quantizer), timed
    # apart from training; training's own root build is st["root_ms"]
    algo_root = args.rows * (F + GH)
    root_gbs = algo_root / (root_mean_ms * 1e-3) / 1e9
    root_merged_gbs = algo_root / (root_merged_ms * 1e-3) / 1e9
    extra = {}
    if st:
        # the histograms accumulated (root + every expansion's smaller child)
        # over the kernels that accumulate them
        acc_bytes = st["root_bytes"] + st["accum_bytes"]
        acc_ms = st["root_ms"] + st["accum_ms"]
        value = acc_bytes / (acc_ms * 1e-3) / 1e9
        launches = max(1.0, st["expand_launches"])
        kernel_gbs = st["accum_bytes"] / (st["accum_ms"] * 1e-3) / 1e9
        kernel_avg_ms = st["accum_ms"] / launches
        part_bytes = st["partition_bytes"]
        per_tree = 1.0 / max(1, stat_steps)
        extra = {
            "hist_rows_features_per_s": round(acc_bytes / (F + GH) * F / (acc_ms * 1e-3), 1),
            "hist_gbs_committed_over_growth": round(st["hist_bytes"] / (st["growth_ms"] * 1e-3) / 1e9, 2),
            "hist_builds_per_tree": round(st["hist_builds"] * per_tree, 2),
            "growth_ms_per_tree": round(st["growth_ms"] * per_tree, 4),
            "accumulation_ms_per_tree": round(acc_ms * per_tree, 4),
            "partition_ms_per_tree": round(st["partition_ms"] * per_tree, 4),
            "partition_gbs": round(part_bytes / (st["partition_ms"] * 1e-3) / 1e9, 2),
            "scan_plan_ms_per_tree": round((st["growth_ms"] - st["root_ms"] - st["partition_ms"]
                                            - st["accum_ms"]) * per_tree, 4),
            "expansion_iterations_per_tree": round(st["iterations"] * per_tree, 2),
            "leaves_expanded_per_tree": round(st["expansions"] * per_tree, 2),
            "rows_accumulated_per_tree": round(st["rows_built"] * per_tree, 1),
            "rows_partitioned_per_tree": round(st["rows_parted"] * per_tree, 1),
            "speculative_row_overhead": round(
                st["rows_built"] / max(1.0, st["hist_bytes"] / (F + GH) - st["root_bytes"] / (F + GH))
                - 1.0, 4),
            "accum_kernel_avg_ms": round(kernel_avg_ms, 5),
            # the root build training runs (quantizing when the lattice is
            # max-abs), BASELINE bytes only, and the quantizer's bytes apart
            "root_build_in_training_ms": round(st["root_ms"] * per_tree, 4),
            "root_build_in_training_gbs": round(st["root_bytes"] / (st["root_ms"] * 1e-3) / 1e9, 1),
            "root_quantizer_bytes_per_tree": round(st["root_quantizer_bytes"] * per_tree, 1),
            "accum_gbs": round(kernel_gbs, 1),
            "accum_size_classes": size_classes(launch_log, 3, 5, F + GH),
        }
        rec_mode = st["partition_bytes"] != st["rows_parted"] * 9.0
        part_row_bytes = st["partition_bytes"] / max(1.0, st["rows_parted"])
        if args.launch_table:
            with open(args.launch_table, "w") as fh:
                fh.write(f"Workload {args.workload}, {stat_steps} trees, leaf rows as "
                         f"{'records' if rec_mode else 'row ids'}; algorithmic bytes per accumulated row "
                         f"F + {GH} = {F + GH}, per partitioned row {part_row_bytes:.1f}\n\n")
                fh.write(size_table_md("k_accum (accumulation) by rows accumulated per launch",
                                       size_classes(launch_log, 3, 5, F + GH)))
                fh.write("\n")
                fh.write(size_table_md("k_partition by rows partitioned per launch",
                                       size_classes(launch_log, 2, 4, part_row_bytes)))
        how = ("streamed from the leaf's records" if args.partition_mode == 1
               else "gathered through the partitioned row list")
        note = (f"dominant histogram kernel k_accum (smaller-child accumulation, {how}) "
                f"over the instrumented {stat_steps}-step training, "
                f"algorithmic bytes per launch = accumulated rows * (F + {GH}) "
                f"({st['accum_bytes'] / launches / 1e6:.2f} MB), over its average kernel duration "
                f"({kernel_avg_ms * 1e3:.1f} us, {int(st['expand_launches'])} launches incl. empty "
                f"tail launches); training's root build "
                f"{st['root_bytes'] / (st['root_ms'] * 1e-3) / 1e9:.0f} GB/s on F + {GH} bytes per row")
    else:
        value = root_gbs
        kernel_gbs = root_gbs
        note = "root build only (instrumented run skipped)"
    out = {
        "metric": METRICS[args.workload],
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / max(1, args.steps), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic",
        "config": {"workload": wl["desc"], "rows": args.rows, "features": F, "max_bin": NB,
                   "num_leaves": L, "steps": args.steps, "trees_per_step": K},
        "train_seconds": round(wall, 3),
        f"train_sec_per_{full}_{'rounds' if K > 1 else 'trees'}": round(full_wall, 3),
        "full_training_trees_kept": full_fit.n_trees,
        "hist_frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        **extra,
        # k_hist over pairs already stored (not the quantizing build that
        # training runs: root_build_in_training_*), alone and with its merge
        "root_hist_stored_pairs_gbs": round(root_gbs, 1),
        "root_hist_stored_pairs_ms": round(root_mean_ms, 4),
        "root_hist_stored_pairs_merged_gbs": round(root_merged_gbs, 1),
        "root_hist_stored_pairs_merged_ms": round(root_merged_ms, 4),
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_per_launch(args.workload + ("rec" if args.partition_mode == 1 else "")),
                     "note": note},
        "cpu_baseline": cpu,
        "records_layout": alt,
        "parity_first_trees_bit_exact": parity,
        "binning": binning,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
