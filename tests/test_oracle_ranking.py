"""Pins the oracle's LambdaRank (src/mojotrees/ranking.mojo:235-771) with the
reference's own ranking tests (tests/test_ranking.mojo), restated on the same
inputs: the hand-calculated lambdas and hessians (within the reference's
1e-8, which is where it pins Mojo's log2), the exact identities those tests
assert between them, truncation, the per-query normalizer, antisymmetry,
isolation of queries, and a ranker that learns a perfect ranking."""
import math

import numpy as np
import pytest

import oracle_lib as O


def _close(a, b, tol=1e-8):
    # tests/test_ranking.mojo:47-48
    return abs(a - b) <= tol * (1.0 + abs(b))


def _log2(x):
    return O.lib().orc_log2(float(x))


def test_log2_and_discounts():
    # exact at powers of two; the discounts of ranks 0..3
    # (tests/test_ranking.mojo:40-44) to the reference's tolerance
    for k in range(-4, 40):
        assert _log2(2.0 ** k) == float(k)
    for x in (3.0, 5.0, 1.5, 1000.0, 1.0 + 1e-6):
        assert abs(_log2(x) - math.log2(x)) <= 1e-9 * abs(math.log2(x))
    want = [1.0, 0.6309297535714575, 0.5, 0.43067655807339306]
    for r, d in enumerate(want):
        assert _close(1.0 / _log2(r + 2.0), d)


def test_single_pair_lambdas_hand_calculated():
    # test_ranking.mojo:310-336
    g, h = O.lambdarank([0.0, 0.0], [1, 0], [2], truncation=30, sigma=1.0, norm=False)
    dn = 1.0 - 1.0 / _log2(3.0)
    assert g[0] == -0.5 * dn and g[1] == 0.5 * dn
    assert h[0] == 0.25 * dn and h[1] == 0.25 * dn
    assert _close(g[0], -0.18453512321427123)
    assert _close(h[0], 0.09226756160713562)


def test_norm_rescales_the_query_hand_calculated():
    # test_ranking.mojo:339-360: equal scores skip the per-pair division, the
    # query factor log2(1 + S) / S applies
    g, h = O.lambdarank([0.0, 0.0], [1, 0], [2], truncation=30, sigma=1.0, norm=True)
    dn = 1.0 - 1.0 / _log2(3.0)
    s = 2.0 * 0.5 * dn
    factor = _log2(1.0 + s) / s
    assert g[0] == -0.5 * dn * factor
    assert h[0] == 0.25 * dn * factor
    assert _close(g[0], -0.22659823629063455)
    assert _close(h[0], 0.11329911814531728)


@pytest.mark.parametrize("scores,labels", [([0.0, 5.0, 0.0], [2, 2, 2]),   # equal labels
                                           ([0.1, 0.2, 0.3], [0, 0, 0]),   # no attainable DCG
                                           ([0.7], [3])])                  # one document
def test_queries_without_pairs_have_zero_lambdas(scores, labels):
    # test_ranking.mojo:363-395
    g, h = O.lambdarank(scores, labels, [len(scores)])
    assert np.all(g == 0.0) and np.all(h == 0.0)


def test_truncation_level_drops_deep_pairs():
    # test_ranking.mojo:398-445
    full_g, full_h = O.lambdarank([0.0] * 3, [2, 1, 0], [3], truncation=30, norm=False)
    assert _close(full_g[0], -0.3082048737868866)
    assert _close(full_g[1], 0.0836164261630733)
    assert _close(full_g[2], 0.22458844762381333)
    assert _close(full_h[0], 0.1541024368934433)
    g, h = O.lambdarank([0.0] * 3, [2, 1, 0], [3], truncation=1, norm=False)
    pair01 = (1.0 - 1.0 / _log2(3.0)) * (1.0 / 3.0)
    assert g[0] == -(pair01 + 0.25) and g[1] == pair01 and g[2] == 0.25
    assert _close(g[0], -0.3730234154761808)
    assert _close(g[1], 0.12302341547618082)
    assert g[1] != full_g[1] and h[2] != full_h[2]


def test_lambdas_are_antisymmetric_and_push_relevant_documents_up():
    # test_ranking.mojo:448-475
    scores = [0.3, -0.2, 1.4, 0.0, 0.9, 0.5, -1.0]
    labels = [1, 3, 0, 2, 0, 4, 1]
    g, h = O.lambdarank(scores, labels, [4, 3])
    for a, b in ((0, 4), (4, 7)):
        assert abs(g[a:b].sum()) < 1e-12
        assert np.all(h[a:b] >= 0.0)
    g, _ = O.lambdarank([0.0] * 3, [0, 1, 2], [3])
    assert g[2] < 0.0 and g[0] > 0.0


def test_queries_do_not_mix():
    # test_ranking.mojo:478-510
    g1, h1 = O.lambdarank([0.4, 0.1, 0.9], [2, 0, 1], [3])
    g2, h2 = O.lambdarank([0.4, 0.1, 0.9] * 2, [2, 0, 1] * 2, [3, 3])
    assert np.array_equal(g2[:3], g1) and np.array_equal(g2[3:], g1)
    assert np.array_equal(h2[:3], h1) and np.array_equal(h2[3:], h1)
    g3, h3 = O.lambdarank([0.4, 0.1, 0.9, 7.0, -7.0, 2.5], [2, 0, 1, 4, 4, 0], [3, 3])
    assert np.array_equal(g3[:3], g1) and np.array_equal(h3[:3], h1)


def test_invalid_ranking_inputs_are_rejected():
    with pytest.raises(ValueError):
        O.lambdarank([0.0, 0.0], [1, 31], [2])
    with pytest.raises(ValueError):
        O.lambdarank([0.0, 0.0], [1, 0], [2], truncation=0)
    with pytest.raises(ValueError):
        O.lambdarank([0.0, 0.0], [1, 0], [2], sigma=0.0)


def ndcg(scores, labels, counts, k):
    """Mean NDCG@k over queries (ranking.ndcg_at_cutoffs, ranking.mojo:326-369)."""
    total, a = 0.0, 0
    for c in counts:
        s, lab = np.asarray(scores[a:a + c]), np.asarray(labels[a:a + c])
        order = sorted(range(c), key=lambda i: -s[i])          # stable
        gains = sorted(lab, reverse=True)
        m = min(k, c)
        dcg = sum((2 ** int(lab[order[j]]) - 1) / _log2(j + 2.0) for j in range(m))
        best = sum((2 ** int(gains[j]) - 1) / _log2(j + 2.0) for j in range(m))
        total += dcg / best if best > 0 else 1.0
        a += c
    return total / len(counts)


def _ranking_dataset(n_queries):
    # test_ranking.mojo:585-600: one feature = relevance (+0.25 on odd
    # queries), rows not sorted by it
    feats, labels = [], []
    for q in range(n_queries):
        for rel in (0, 3, 1, 2):
            feats.append(rel + 0.25 * (q % 2))
            labels.append(rel)
    return np.array(feats), np.array(labels, np.float64), [4] * n_queries


def _train_ranker(n_queries, rounds):
    x, y, counts = _ranking_dataset(n_queries)
    n = len(y)
    bins = O.bin_equal_width(x, n, 1, 8)
    p, st = O.rank_params(counts, num_iterations=rounds, learning_rate=0.3, num_leaves=8,
                          min_data_in_leaf=1, lambda_l2=1.0, min_sum_hessian=1e-3,
                          use_quantized_grad=0)
    m = O.train(bins, n, 1, 8, y, p)
    return m, bins, y, counts, st


def test_training_learns_a_perfect_ranking():
    # test_ranking.mojo:604-624
    m, bins, y, counts, _ = _train_ranker(6, 60)
    n = len(y)
    assert ndcg(np.zeros(n), y, counts, 4) < 0.95
    assert m.n_trees > 0 and m.base[0] == 0.0
    raw, _ = m.predict_binned(bins, n, 1)
    assert ndcg(raw, y, counts, 4) == 1.0 and ndcg(raw, y, counts, 1) == 1.0
    assert np.array_equal(raw, m.train_raw(n))


def test_training_is_deterministic():
    # test_ranking.mojo:627-638
    a, bins, y, _, _ = _train_ranker(5, 25)
    b, _, _, _, _ = _train_ranker(5, 25)
    assert a.n_trees == b.n_trees
    assert np.array_equal(a.train_raw(len(y)), b.train_raw(len(y)))


def test_training_rejects_bad_labels_and_groups():
    # test_ranking.mojo:641-660
    x, y, counts = _ranking_dataset(2)
    bins = O.bin_equal_width(x, 8, 1, 8)
    bad = y.copy()
    bad[0] = 31
    p, st = O.rank_params(counts, num_iterations=3)
    with pytest.raises(RuntimeError):
        O.train(bins, 8, 1, 8, bad, p)
    p, st = O.rank_params([4, 3], num_iterations=3)       # 7 rows for 8
    with pytest.raises(RuntimeError):
        O.train(bins, 8, 1, 8, y, p)
