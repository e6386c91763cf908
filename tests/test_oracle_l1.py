"""L1 regularization in the oracle (gain.soft_threshold_l1 / leaf_score,
src/mojotrees/gain.mojo:17-35; tree._leaf_value, tree.mojo:1961-1995),
pinned without the reference:

- the split search under lambda_l1 > 0 equals an exhaustive enumeration of
  every candidate scored with the closed form T(G)^2 / (H + l2), T the soft
  threshold sign(G) max(|G| - l1, 0), parent term included;
- a node whose |G| is at most lambda_l1 has leaf value exactly 0, and a
  lambda_l1 above every node's |G| grows single-leaf trees of value 0;
- a stump's two leaf values equal -T(G) / (H + l2) with G, H summed by brute
  force over the rows each leaf holds (quantized: the dequantized integer
  sums), so a dropped or mis-signed threshold fails.
"""
import numpy as np
import pytest

import oracle_lib as O
from test_oracle_quantized import _brute_split


def _soft(g, l1):
    return np.sign(g) * max(abs(g) - l1, 0.0)


def _brute_split_l1(hist, missing_bin, widths, gu, hu, l1, l2, min_hess, min_data):
    """_brute_split with the soft-thresholded score."""

    nf, nb, _ = hist.shape
    hmin = int(np.ceil(min_hess * hu)) if min_hess > 0 else 0

    def score(g, h):
        t = _soft(g / gu, l1)
        return t * t / (h / hu + l2)

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


@pytest.mark.parametrize("seed", range(10))
@pytest.mark.parametrize("l1", [0.05, 0.4, 3.0])
def test_quantized_split_under_l1_matches_brute_force(seed, l1):
    rng = np.random.default_rng(500 + seed)
    nf, nb = 4, 9
    n = int(rng.integers(30, 400))
    bins = rng.integers(0, nb, size=(nf, n), dtype=np.uint8)
    qg = rng.integers(-2, 3, size=n).astype(np.int8)
    qh = rng.integers(0, 5, size=n).astype(np.int8)
    missing = np.full(nf, -1, np.int32)
    if seed % 3 == 1:
        missing[1] = nb - 1
    widths = np.array([max(int(bins[f].max()) + 1, missing[f] + 1) for f in range(nf)], np.int32)
    h = O.hist_quantized(bins.ravel(), n, nf, nb, qg, qh)
    gu, hu = 2.0 / 0.37, 4.0 / 0.25
    md = int(rng.integers(1, 12))
    found, f, b, dl, gain = O.split_quantized(h, missing, widths, gu, hu, l1, 1.0, 1e-3, md)
    want = _brute_split_l1(h, missing, widths, gu, hu, l1, 1.0, 1e-3, md)
    if want is None:
        assert not found
    else:
        assert found and (f, b, dl) == want[1:] and gain == pytest.approx(want[0], rel=1e-12)
    # with l1 = 0 the soft threshold is the identity: the plain enumeration
    if l1 == 0.05:
        f0 = O.split_quantized(h, missing, widths, gu, hu, 0.0, 1.0, 1e-3, md)
        w0 = _brute_split(h, missing, widths, gu, hu, 1.0, 1e-3, md)
        assert (w0 is None) == (not f0[0])


@pytest.mark.parametrize("quantized", [0, 1])
def test_l1_above_every_gradient_sum_gives_zero_leaves(quantized):
    rng = np.random.default_rng(3)
    n, f = 3000, 4
    x = rng.normal(size=(f, n))
    y = x[0] + 0.5 * x[1] + 0.1 * rng.normal(size=n)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=32)
    # the root's |G| = |sum(raw - y)| is at most sum |y - mean| < 10 n
    m = O.train(bins, n, f, 32, y, O.default_params(objective=0, num_iterations=3, num_leaves=15,
                                                    lambda_l1=10.0 * n, use_quantized_grad=quantized),
                missing_bin=mb)
    for t in range(m.n_trees):
        tr = m.tree(t)
        assert len(tr["feature"]) == 1 and tr["feature"][0] < 0
        assert tr["value"][0] == 0.0


@pytest.mark.parametrize("quantized", [0, 1])
@pytest.mark.parametrize("l1", [0.0, 2.5, 40.0])
def test_stump_leaf_values_are_the_soft_thresholded_closed_form(quantized, l1):
    rng = np.random.default_rng(int(l1 * 10) + quantized)
    n, f = 2000, 3
    x = rng.normal(size=(f, n))
    y = (x[0] > 0.3).astype(np.float64) * 2.0 + 0.2 * rng.normal(size=n)
    bins, _, _, mb = O.fit_transform(x.ravel(), n, f, max_bins=16)
    l2 = 1.0
    p = O.default_params(objective=0, num_iterations=1, num_leaves=2, lambda_l1=l1, lambda_l2=l2,
                         min_data_in_leaf=5, use_quantized_grad=quantized, stochastic_rounding=0)
    m = O.train(bins, n, f, 16, y, p, missing_bin=mb)
    tr = m.tree(0)
    assert tr["feature"][0] >= 0, "the stump must split"
    fe, thr = int(tr["feature"][0]), int(tr["threshold"][0])
    col = bins.reshape(f, n)[fe]
    left = col <= thr
    base = float(m.base[0])
    g, h = O.grad_hess(0, np.full(n, base), y)
    if quantized:
        qg, qh, sc = O.quantize_rule(g, h, O.RULE_MAX_ABS, stochastic=0, const_hessian=1)
        G = lambda sel: float(qg[sel].astype(np.int64).sum()) / sc[0]
        H = lambda sel: float(qh[sel].astype(np.int64).sum()) / sc[1]
    else:
        G = lambda sel: float(np.sum(g[sel]))
        H = lambda sel: float(np.sum(h[sel]))
    for child, sel in ((tr["left"][0], left), (tr["right"][0], ~left)):
        want = -_soft(G(sel), l1) / (H(sel) + l2)
        assert tr["value"][child] == pytest.approx(want, rel=1e-12, abs=1e-300)
