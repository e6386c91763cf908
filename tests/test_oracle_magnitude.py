"""The oracle's magnitude-sum lattice, pinned without the reference.

What fixes each function:
- largest_power_of_two_at_most (quantized_gradient.mojo:856-888): closed
  forms -- an exact power maps to itself, every value inside a binade maps to
  its bottom (checked against math.frexp), zero, negatives, non-finite values
  and subnormals are refused.
- fixed_point_scale_pow2 (:908-1117): the reference's own assertions
  (tests/test_cpu_quantized_grad.mojo:429-460): the factor is its own power-of-
  two floor and at most 2^30 / sum|g|; plus more than half of it (a floor,
  not a round), hand-computed values, the magnitude floor, and the binary32
  refusal below 2^-149.
- magnitude_sums (gpu_objectives_native._abs_sum_kernel :982-1040 and
  sum_abs_partials :1100-1125): one input whose binary32 total depends on the
  exact order -- thread t of workgroup b taking rows b*256 + t + k*65536, the
  workgroup's halving tree, the binary64 fold -- and whose expected total is
  derived by hand below; a sequential binary32 sum, a binary64 sum and a
  different stride all give other numbers.
- the max-abs arm's units as the reference asserts them
  (tests/test_cpu_quantized_grad.mojo:384-426).
"""
import math

import numpy as np
import pytest

import oracle_lib as O


@pytest.mark.parametrize("k", list(range(-1022, 1024, 37)) + [-1022, 0, 1, 30, 1023])
def test_power_of_two_floor_closed_forms(k):
    p = math.ldexp(1.0, k)
    assert O.largest_power_of_two_at_most(p) == p
    for m in (1.0000001, 1.25, 1.5, 1.9999999):
        x = m * p
        if math.isfinite(x):
            fr, e = math.frexp(x)
            assert O.largest_power_of_two_at_most(x) == math.ldexp(1.0, e - 1) == p


@pytest.mark.parametrize("x", [0.0, -1.0, -0.0, math.inf, math.nan, 5e-324, 2.0 ** -1030])
def test_power_of_two_floor_refusals(x):
    assert O.largest_power_of_two_at_most(x) == -1.0


def test_pow2_scale_is_the_reference_rule():
    rng = np.random.default_rng(8)
    for total in list(rng.lognormal(3.0, 6.0, 300)) + [1.0, 3.0, 2.0 ** 30, 2.0 ** 30 + 1]:
        s = O.fixed_point_scale_pow2(total)
        # tests/test_cpu_quantized_grad.mojo:449-460
        assert s == O.largest_power_of_two_at_most(s)
        assert s <= 2.0 ** 30 / total
        # a floor: the next power up would exceed the quotient
        assert 2.0 * s > 2.0 ** 30 / total
        assert float(np.float32(s)) == s
    assert O.fixed_point_scale_pow2(1.0) == 2.0 ** 30
    assert O.fixed_point_scale_pow2(3.0) == 2.0 ** 28          # 2^30 / 3 = 3.58e8
    assert O.fixed_point_scale_pow2(2.0 ** 30) == 1.0
    assert O.fixed_point_scale_pow2(2.0 ** 30 + 1.0) == 0.5
    # an exact power of two quotient is kept, not rounded one binade down
    assert O.fixed_point_scale_pow2(2.0 ** 10) == 2.0 ** 20
    # all-zero gradients: the total floors at 1e-12, 2^30 / 1e-12 = 1.07e21
    # lies in [2^69, 2^70)
    assert O.fixed_point_scale_pow2(0.0) == 2.0 ** 69
    assert O.fixed_point_scale_pow2(1e-13) == 2.0 ** 69
    # the smallest binary32 power is 2^-149: 2^30 / 2^178 = 2^-148 is kept,
    # 2^30 / 2^180 = 2^-150 would round up and is refused
    assert O.fixed_point_scale_pow2(2.0 ** 178) == 2.0 ** -148
    assert O.fixed_point_scale_pow2(2.0 ** 180) == -1.0
    assert O.fixed_point_scale_pow2(math.inf) == -1.0
    assert O.fixed_point_scale_pow2(math.nan) == -1.0


def test_magnitude_sum_order_hand_derived():
    """n = 3 * 65536 rows, |g| = 2^24 on row 0 and 1 elsewhere.

    Thread 0 of workgroup 0 adds rows 0, 65536, 131072 in binary32:
    2^24 + 1 rounds to 2^24 (ties to even), twice, so it holds 2^24; every
    other thread holds 3. Workgroup 0 halves its 256 sums: 2^24 + 3 =
    16777219 rounds to 16777220 (spacing 2 at 2^24, tie to the even
    significand); then it adds 6, 12, 24, 48, 96, 192, 384 exactly:
    16777982. The other 255 workgroups sum to 768 each. The binary64 fold:
    16777982 + 255 * 768 = 16973822. The exact sum is 16973823; a sequential
    binary32 sum stays at 2^24 + a few."""
    n = 3 * 65536
    g = np.ones(n)
    g[0] = 2.0 ** 24
    h = np.full(n, 0.5)
    sg, sh = O.magnitude_sums(g, h)
    assert sg == 16973822.0
    assert sg != float(np.sum(g))                    # binary64 sum: 16973823
    seq = np.float32(0.0)
    for v in g[:1000].astype(np.float32):
        seq = np.float32(seq + v)
    assert seq == np.float32(2.0 ** 24)              # a sequential sum loses the ones
    assert sh == 0.5 * n                             # exact: every partial is a small dyadic
    # the sample excludes row 0: thread 0 of workgroup 0 adds two ones
    mask = np.ones(n, np.uint8)
    mask[0] = 0
    assert O.magnitude_sums(g, h, mask) == (float(n - 1), 0.5 * (n - 1))
    # a row whose hessian is not finite adds to neither sum. Row 7 leaves
    # thread 7 with 2: the halving carries 5, 11, 23, 47, 95 down to thread
    # 7, which a = 4 adds into thread 3 (96 + 95 = 191) and a = 2 into thread
    # 1 (192 + 191 = 383); thread 0 then holds 16777598 + 383 = 16777981,
    # a tie that rounds to the even 16777980: 16777980 + 255 * 768.
    h2 = h.copy()
    h2[7] = np.inf
    assert O.magnitude_sums(g, h2) == (16973820.0, 0.5 * (n - 1))


def test_magnitude_sum_close_to_binary64():
    rng = np.random.default_rng(3)
    g = rng.normal(size=300_001).astype(np.float32).astype(np.float64)
    h = rng.uniform(0.0, 0.25, size=300_001).astype(np.float32).astype(np.float64)
    sg, sh = O.magnitude_sums(g, h)
    assert abs(sg - np.abs(g).sum()) <= 1e-6 * np.abs(g).sum()
    assert abs(sh - h.sum()) <= 1e-6 * h.sum()


@pytest.mark.parametrize("stochastic", [0, 1])
def test_magnitude_sum_quantizer(stochastic):
    rng = np.random.default_rng(12 + stochastic)
    n = 50_000
    g = rng.normal(size=n).astype(np.float32).astype(np.float64)
    h = rng.uniform(0.01, 0.25, size=n).astype(np.float32).astype(np.float64)
    qg, qh, sc = O.quantize_rule(g, h, O.RULE_MAGNITUDE_SUM, stochastic=stochastic)
    sg, sh = O.magnitude_sums(g, h)
    assert sc[0] == O.fixed_point_scale_pow2(sg) and sc[1] == O.fixed_point_scale_pow2(sh)
    assert sc[2] == sc[3] == 2.0 ** 30
    y = g * sc[0]                                    # exact: a power-of-two factor
    if stochastic:
        assert np.all(np.abs(qg - y) < 1.0)
        assert np.all(np.sign(qg) * np.sign(y) >= 0)
    else:
        # round half away from zero
        assert np.array_equal(qg, (np.sign(y) * np.floor(np.abs(y) + 0.5)).astype(np.int64))
    # the headroom argument: the lattice total stays within 2^30 + n
    assert np.abs(qg.astype(np.int64)).sum() <= 2 ** 30 + n
    assert np.abs(qh.astype(np.int64)).sum() <= 2 ** 30 + n
    # a constant hessian takes LightGBM's one-unit lattice under both rules
    qg2, qh2, sc2 = O.quantize_rule(g, np.ones(n), O.RULE_MAGNITUDE_SUM, stochastic=stochastic,
                                    const_hessian=1)
    assert sc2[1] == 1.0 and sc2[3] == 1.0 and np.all(qh2 == 1)
    assert np.array_equal(qg2, qg)


@pytest.mark.parametrize("B", [2, 4, 16, 126])
def test_max_abs_units_are_lightgbms(B):
    """tests/test_cpu_quantized_grad.mojo:384-426: units = (B / 2) / max|g|
    and B / max|h|, one unit over max|h| for a constant hessian."""
    rng = np.random.default_rng(B)
    g = rng.normal(size=300)
    h = rng.uniform(0.1, 2.0, size=300)
    _, _, sc = O.quantize_rule(g, h, O.RULE_MAX_ABS, quant_bins=B)
    assert sc[0] == (B / 2) / np.abs(g).max()
    assert sc[1] == B / np.abs(h).max()
    assert sc[2] == B // 2 and sc[3] == B
    _, qh, sc = O.quantize_rule(g, np.ones(300), O.RULE_MAX_ABS, quant_bins=B, const_hessian=1)
    assert sc[1] == 1.0 and sc[3] == 1 and np.all(qh == 1)


def test_int32_histogram_is_the_scatter_add():
    rng = np.random.default_rng(4)
    n, f, nb = 5000, 5, 17
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    qg = rng.integers(-2 ** 30, 2 ** 30, size=n).astype(np.int32)
    qh = rng.integers(0, 2 ** 20, size=n).astype(np.int32)
    rows = np.sort(rng.choice(n, 1234, replace=False)).astype(np.int32)
    got = O.hist_quantized32(bins.ravel(), n, f, nb, qg, qh, rows)
    want = np.zeros((f, nb, 3), np.int64)
    for j in range(f):
        np.add.at(want[j, :, 0], bins[j, rows], qg[rows].astype(np.int64))
        np.add.at(want[j, :, 1], bins[j, rows], qh[rows].astype(np.int64))
        np.add.at(want[j, :, 2], bins[j, rows], 1)
    assert np.array_equal(got, want)
