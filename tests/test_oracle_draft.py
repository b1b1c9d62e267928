"""Pins of the draft-side oracle functions (CPU only).

Closed forms and brute force for what the reference's draft step decides
(single/eval_sync.py): the top-k filter of _sampling_probs (:292-295, ties
with the k-th value kept), the nucleus filter of _sample_with_sparse_probs
(:356-361), _select_transfer with plain and "dynamic" remasking (:447-465),
the one-hot greedy confidence (:287-291, :323-338) and the transfer
schedule (:440-444).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def test_topk_keep_keeps_ties_with_the_kth_value():
    x = np.array([1.0, 5.0, 3.0, 5.0, 3.0, 3.0, -2.0], np.float32)
    # sorted descending: 5 5 3 3 3 1 -2
    assert oracle.topk_keep(x, 1.0, 1).tolist() == [False, True, False, True, False, False, False]
    assert oracle.topk_keep(x, 1.0, 2).tolist() == [False, True, False, True, False, False, False]
    assert oracle.topk_keep(x, 1.0, 3).tolist() == [False, True, True, True, True, True, False]
    assert oracle.topk_keep(x, 1.0, 0).all()
    assert oracle.topk_keep(x, 1.0, 100).all()


def test_topk_keep_compares_the_fp32_quotient():
    """Two logits that differ in fp32 but divide to the same fp32 quotient are
    both kept at k = 1: the reference filters logits.float() / T."""
    T = np.float32(0.75)
    a = np.float32(1.6)
    b = np.nextafter(a, np.float32(2))  # quotients above 2 are spaced 2^-22 apart
    assert a != b and a / T == b / T
    x = np.array([a, b, 0.5], np.float32)
    assert oracle.topk_keep(x, float(T), 1).tolist() == [True, True, False]


def test_softmax_rows_closed_form():
    x = np.log(np.array([[1.0, 2.0, 3.0, 4.0]], np.float32))
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0)[0], [0.1, 0.2, 0.3, 0.4], rtol=1e-6)
    # top-2 keeps {3, 4}: 3/7, 4/7
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0, top_k=2)[0], [0, 0, 3 / 7, 4 / 7], rtol=1e-6)
    # T = 0.5 squares the ratios
    np.testing.assert_allclose(oracle.softmax_rows(x, 0.5)[0], np.array([1, 4, 9, 16]) / 30, rtol=1e-5)
    # greedy: one-hot at the first maximum
    y = np.array([[0.0, 2.0, 2.0, 1.0]], np.float32)
    assert oracle.softmax_rows(y, 0.0)[0].tolist() == [0.0, 1.0, 0.0, 0.0]


def test_sample_with_prob_top_k_draws_only_kept_entries():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(64, 300)).astype(np.float32)
    u = rng.random(64)
    tok, prob, _ = oracle.sample_with_prob(x, 0.7, u, top_k=5)
    for n in range(64):
        keep = oracle.topk_keep(x[n], 0.7, 5)
        assert keep[tok[n]]
        z = x[n][keep].astype(np.float64) / 0.7
        e = np.exp(z - z.max())
        np.testing.assert_allclose(prob[n], np.exp(x[n][tok[n]] / 0.7 - z.max()) / e.sum(), rtol=1e-6)


def test_sparse_top_p_closed_form():
    # Support logits log(0.5), log(0.3), log(0.2): inclusive sums 0.5, 0.8, 1.0.
    x = np.full((1, 10), -50.0, np.float32)
    x[0, 3], x[0, 7], x[0, 1] = np.log(0.5), np.log(0.3), np.log(0.2)
    _, ids, probs, _ = oracle.sample_sparse(x, 1.0, 3, [0.1], top_p=0.6)
    assert ids[0].tolist() == [3, 7, 1]
    # entry 2 goes (0.8 > 0.6); entry 1 stays (0.5 <= 0.6)
    np.testing.assert_allclose(probs[0], [0.5 / 0.8, 0.3 / 0.8, 0.0], rtol=1e-6)
    _, _, probs, _ = oracle.sample_sparse(x, 1.0, 3, [0.1], top_p=0.4)
    np.testing.assert_allclose(probs[0], [1.0, 0.0, 0.0], rtol=1e-12)
    _, _, probs, _ = oracle.sample_sparse(x, 1.0, 3, [0.1], top_p=1.0)
    np.testing.assert_allclose(probs[0], [0.5, 0.3, 0.2], rtol=1e-6)


@pytest.mark.parametrize("dynamic", [False, True])
def test_select_transfer_brute_force(dynamic):
    """Against an independent ranking: sort masked positions by (-conf,
    position) and take the first kk."""
    rng = np.random.default_rng(1)
    M = 99
    for trial in range(200):
        Q = int(rng.integers(1, 24))
        blk = np.where(rng.random((1, Q)) < 0.6, M, rng.integers(0, 50, (1, Q)))
        x0 = rng.integers(0, 50, (1, Q))
        conf = np.round(rng.random((1, Q)), 1).astype(np.float32)  # many ties
        k = int(rng.integers(0, Q + 2))
        thr = float(rng.choice([0.0, 0.5, 0.95, 2.0]))
        got, sel = oracle.select_transfer(blk, M, k, x0, conf, dynamic=dynamic, threshold=thr)
        masked = [i for i in range(Q) if blk[0, i] == M]
        n_conf = sum(conf[0, i] >= np.float32(thr) for i in masked)
        kk = min(k, n_conf) if dynamic and n_conf > 0 else k
        order = sorted(masked, key=lambda i: (-conf[0, i], i))[:kk]
        want = blk.copy()
        want[0, order] = x0[0, order]
        np.testing.assert_array_equal(got, want)
        assert sorted(np.nonzero(sel[0])[0].tolist()) == sorted(order)


def test_dynamic_remasking_cases():
    M = 7
    blk = np.array([[M, M, M, M, M, 3]])
    x0 = np.array([[10, 11, 12, 13, 14, 15]])
    conf = np.array([[0.2, 0.95, 0.3, 0.91, 0.1, 0.99]], np.float32)
    # two masked positions reach 0.9: only they are unmasked, even with k = 4
    got, _ = oracle.select_transfer(blk, M, 4, x0, conf, dynamic=True, threshold=0.9)
    assert got.tolist() == [[M, 11, M, 13, M, 3]]
    # k = 1 takes the more confident of the two
    got, _ = oracle.select_transfer(blk, M, 1, x0, conf, dynamic=True, threshold=0.9)
    assert got.tolist() == [[M, 11, M, M, M, 3]]
    # none reaches the threshold: plain top-k
    got, _ = oracle.select_transfer(blk, M, 2, x0, conf, dynamic=True, threshold=0.999)
    assert got.tolist() == [[M, 11, M, 13, M, 3]]


def test_one_hot_confidence_takes_the_lowest_masked_positions():
    rng = np.random.default_rng(3)
    B, Q, V, M = 3, 16, 50, 49
    x = rng.normal(size=(B, Q, V)).astype(np.float32)
    blk = np.full((B, Q), M)
    blk[0, :3] = 1
    blk[1, [2, 5, 9]] = 1
    got, x0, conf = oracle.confidence_topk(x, blk, M, 4, 0.0, one_hot=True)
    assert (conf == 1.0).all()
    for b in range(B):
        masked = [i for i in range(Q) if blk[b, i] == M][:4]
        want = blk[b].copy()
        want[masked] = x.argmax(-1)[b, masked]
        np.testing.assert_array_equal(got[b], want)


def test_transfer_schedule():
    assert oracle.num_transfer_tokens(16, 4) == [4, 4, 4, 4]
    assert oracle.num_transfer_tokens(15, 4) == [4, 4, 4, 3]
    assert oracle.num_transfer_tokens(5, 8) == [1, 1, 1, 1, 1, 0, 0, 0]
    assert oracle.num_transfer_tokens(7, 0) == [7]
    for n in range(40):
        for s in range(1, 9):
            sch = oracle.num_transfer_tokens(n, s)
            assert sum(sch) == n and max(sch) - min(sch) <= 1 and sch == sorted(sch, reverse=True)


def test_top_p_filter_closed_form():
    # probabilities 0.4 0.3 0.2 0.1: running sums 0.4 0.7 0.9 1.0
    x = np.log(np.array([[0.1, 0.4, 0.2, 0.3]], np.float32))
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0, top_p=0.5)[0], [0, 0.4 / 0.7, 0, 0.3 / 0.7], rtol=1e-6)
    # 0.4 already exceeds 0.35: only the first entry stays
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0, top_p=0.35)[0], [0, 1, 0, 0], rtol=1e-12)
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0, top_p=0.75)[0], [0, 0.4 / 0.9, 0.2 / 0.9, 0.3 / 0.9],
                               rtol=1e-6)
    # top-k first: {0.4, 0.3} renormalised to 4/7, 3/7; 4/7 > 0.5 keeps one
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0, top_k=2, top_p=0.5)[0], [0, 1, 0, 0], rtol=1e-12)
    np.testing.assert_allclose(oracle.softmax_rows(x, 1.0, top_k=2, top_p=0.6)[0], [0, 4 / 7, 0, 3 / 7], rtol=1e-6)
    keep, margin = oracle.filter_keep(x[0], 1.0, 0, 0.5)
    assert keep.tolist() == [False, True, False, True]
    np.testing.assert_allclose(margin, 0.1, rtol=1e-5)  # |0.4 - 0.5|
    assert oracle.filter_keep(x[0], 1.0, 0, 1.0)[1] == np.inf


def test_top_p_cut_through_ties_keeps_the_lowest_ids():
    x = np.zeros(4, np.float32)  # four equal entries: running sums .25 .5 .75 1
    keep, _ = oracle.filter_keep(x, 1.0, 0, 0.3)
    assert keep.tolist() == [True, True, False, False]
    x = np.array([2.0, 1.0, 1.0, 1.0, 3.0], np.float32)
    p = np.exp(x - 3.0)
    p /= p.sum()
    # order: id 4, id 0, then ids 1, 2, 3 tied
    c = np.cumsum(p[[4, 0, 1, 2, 3]])
    top_p = (c[2] + c[3]) / 2  # between the 1st and 2nd tie: ids 4, 0, 1, 2 stay
    keep, _ = oracle.filter_keep(x, 1.0, 0, float(top_p))
    assert keep.tolist() == [True, True, True, False, True]


def test_top_p_kept_set_is_the_minimal_sorted_prefix():
    """Property pin: the kept set is a prefix of the descending order (ties
    by id) whose mass exceeds top_p while the prefix without its last entry
    does not (or it is everything), checked from the definitions in fp64."""
    rng = np.random.default_rng(11)
    for trial in range(60):
        V = int(rng.integers(2, 400))
        x = np.round(rng.normal(size=V) * 2, int(rng.integers(0, 3))).astype(np.float32)  # with ties
        T = float(rng.choice([1.0, 0.7, 1.3]))
        top_k = int(rng.choice([0, 1, 5, V // 2]))
        top_p = float(rng.uniform(0.05, 0.99))
        keep, _ = oracle.filter_keep(x, T, top_k, top_p)
        base = oracle.topk_keep(x, T, top_k)
        z = x / np.float32(T)
        idx = np.flatnonzero(base)
        order = sorted(idx, key=lambda i: (-float(z[i]), i))
        kept = [i for i in order if keep[i]]
        assert kept == order[:len(kept)] and len(kept) >= 1
        assert not keep[~base].any()
        e = np.exp(z[order].astype(np.float64) - float(z[order[0]]))
        mass = np.cumsum(e / e.sum())
        m = len(kept)
        assert m == len(order) or mass[m - 1] > top_p
        assert m == 1 or mass[m - 2] <= top_p


def test_sample_sparse_ranks_the_fp32_quotient_with_ties_by_id():
    T = np.float32(0.75)
    a = np.float32(1.6)
    b = np.nextafter(a, np.float32(2))  # equal fp32 quotients, different logits
    x = np.array([[0.1, b, a, 0.0]], np.float32)
    _, ids, _, _ = oracle.sample_sparse(x, float(T), 3, [0.5])
    assert ids[0].tolist() == [1, 2, 0]
