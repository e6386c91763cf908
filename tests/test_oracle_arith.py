"""Closed-form and known-answer checks of the oracle's arithmetic.

References: rng (src/mojotrees/rng.mojo:35-46), quant_stream and
quantize_scalar (src/mojotrees/quantized_gradient.mojo:475-492, 1479-1545),
hessian_units_at_least (:3336-3364), Mojo exp/log restatements (pinned
bit-for-bit by the golden fixtures, bounded here against libm).
"""
import math

import numpy as np
import pytest

import golden_fixtures as G
import oracle_lib as O


def test_splitmix64_known_answers():
    L = O.lib()
    # First outputs of the standard SplitMix64 generator seeded with 0: the
    # state advances by the golden gamma before each mix.
    assert L.orc_splitmix64(0) == 0xE220A8397B1DCDAF
    assert L.orc_splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    ks = np.arange(1000, dtype=np.uint64) * np.uint64(7919)
    ref = G.splitmix64(ks)
    got = np.array([L.orc_splitmix64(int(k)) for k in ks], dtype=np.uint64)
    assert np.array_equal(ref, got)


def test_uniform_is_top_53_bits():
    L = O.lib()
    for c in [0, 1, 2, 12345, 2**63 + 5]:
        want = (L.orc_splitmix64(c) >> 11) / 2.0**53
        assert L.orc_uniform(c) == want
        assert 0.0 <= want < 1.0


def test_quant_stream_planes_and_classes_differ():
    L = O.lib()
    g = L.orc_quant_stream(11, 3, 0, 0)
    h = L.orc_quant_stream(11, 3, 0, 1)
    c1 = L.orc_quant_stream(11, 3, 1, 0)
    r4 = L.orc_quant_stream(11, 4, 0, 0)
    assert len({g, h, c1, r4}) == 4
    # closed form: splitmix64 chain over (seed, round, class + 1, plane * GOLDEN)
    sm = L.orc_splitmix64
    want = sm(sm(sm(sm(11) ^ 3) ^ 1) ^ ((1 * 0x9E3779B97F4A7C15) & (2**64 - 1)))
    assert h == want


def test_exp_log_close_to_libm():
    """The reference's exp and log are not correctly rounded (their bits are
    pinned by the golden fixtures); here they are bounded against libm."""
    L = O.lib()
    # The reduction uses ln2 truncated by ~2.8e-13 relative, so the error
    # grows with k = round(x / ln2): |rel err| <= ~4e-13 * (1 + |x|).
    xs = np.linspace(-700, 700, 20001)
    for x in xs:
        e = L.orc_exp(float(x))
        assert abs(e - math.exp(x)) <= 1e-12 * (1.0 + abs(x)) * math.exp(x)
    for x in np.linspace(-0.34, 0.34, 2001):  # k = 0: the polynomial alone
        assert abs(L.orc_exp(float(x)) - math.exp(x)) <= 4e-16 * math.exp(x)
    assert L.orc_exp(0.0) == 1.0
    for x in np.geomspace(1e-15, 1e15, 4001):
        lv = L.orc_log(float(x))
        # single-precision-grade polynomial (Cephes logf) in binary64
        assert abs(lv - math.log(x)) <= 2e-9 * max(1.0, abs(math.log(x)))


def test_sigmoid_branches():
    L = O.lib()
    for x in [-30.0, -2.5, -1e-3, 0.0, 1e-3, 2.5, 30.0]:
        s = L.orc_sigmoid(x)
        assert abs(s - 1.0 / (1.0 + math.exp(-x))) < 1e-12
        assert 0.0 < s < 1.0 or abs(x) > 20


def test_quantize_worked_example_magnitude_symmetric():
    """y = -1.3 with a dither u in (0.7, 1) must round to -2 (LightGBM's
    magnitude-symmetric rule, quantized_gradient.mojo:1502-1505), where
    floor(y + u) would give -1."""
    L = O.lib()
    n = 64
    seed, rnd = 11, 0
    stream = L.orc_quant_stream(seed, rnd, 0, 0)
    us = np.array([L.orc_uniform((stream + r) & (2**64 - 1)) for r in range(n)])
    r_hit = int(np.nonzero((us > 0.7) & (us < 1.0))[0][0])
    grad = np.full(n, 0.25)
    grad[0] = 2.0            # max |g| = 2  ->  grad units = (4/2) / 2 = 1
    grad[r_hit] = -1.3
    hess = np.full(n, 0.5)
    qg, qh, sc = O.quantize(grad, hess, quant_bins=4, stochastic=1, seed=seed,
                            round_index=rnd)
    assert sc[0] == 1.0 and sc[2] == 2
    assert qg[r_hit] == -2
    assert qg[0] == 2


def test_quantize_scales_and_bounds():
    rng = np.random.default_rng(5)
    n = 20000
    g = rng.normal(size=n).astype(np.float32).astype(np.float64)
    h = rng.uniform(0.01, 0.25, size=n).astype(np.float32).astype(np.float64)
    for B in (2, 4, 16, 126):
        qg, qh, sc = O.quantize(g, h, quant_bins=B, stochastic=1, round_index=7)
        gmax, hmax = np.abs(g).max(), np.abs(h).max()
        assert sc[0] == (B // 2) / gmax
        assert sc[1] == B / hmax
        y = g * sc[0]
        assert np.all(np.abs(qg) <= B // 2)
        assert np.all((qh >= 0) & (qh <= B))
        # magnitude rounded to floor or ceil, sign kept
        assert np.all(np.abs(qg - y) < 1.0)
        assert np.all((np.sign(qg) == np.sign(y)) | (qg == 0))
        # unbiased: the rounding error averages to ~0 (B=2: lattice of 2 units)
        assert abs(np.mean(qg - y)) < 0.02


def test_quantize_round_to_nearest_and_const_hessian():
    g = np.array([0.5, -0.5, 0.26, -0.74, 1.0])
    h = np.ones(5)
    qg, qh, sc = O.quantize(g, h, quant_bins=4, stochastic=0, const_hessian=1)
    # units 2: y = 1, -1, 0.52, -1.48, 2 -> round half away from zero
    assert list(qg) == [1, -1, 1, -1, 2]
    assert sc[1] == 1.0 and list(qh) == [1] * 5


def test_quantize_uses_subset_for_scale():
    g = np.array([10.0, 1.0, -0.5, 0.25])
    h = np.array([1.0, 0.5, 0.5, 0.5])
    _, _, full = O.quantize(g, h, stochastic=0)
    _, _, sub = O.quantize(g, h, rows=np.array([1, 2, 3]), stochastic=0)
    assert full[0] == 2 / 10.0 and sub[0] == 2 / 1.0
