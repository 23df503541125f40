"""Pins the CPU restatement of sample() and of Philox4x32-10 (oracle/sampling.py).

Philox is checked against the Random123 known-answer vectors (kat_vectors of the Random123 1.x
distribution).  sample() has no test or fixture in the reference (packages/model-utils has no
sampling test), so its restatement is pinned by cases whose answers follow from the definition by
hand: id-order versus sorted-order draws, top-k / top-p cut-offs on probabilities with closed
forms, greedy ties, the inverse-CDF counts of a grid of r, and the fallback of sampleFromProbs.
"""
import math

import numpy as np
import pytest
from scipy.special import softmax

from oracle.sampling import (draw_from_probs, filtered_probs, philox4x32_10, sample_reference, topp_margin,
                             uniform24)

LN = np.log


@pytest.mark.parametrize("ctr,key,want", [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox_random123_kat(ctr, key, want):
    assert philox4x32_10(ctr, key) == want


def test_uniform24_range_and_key_halves():
    # word 0 of the all-zero KAT, top 24 bits
    assert uniform24(0, 0) == (0x6627e8d5 >> 8) / 2 ** 24
    # the seed's low half is the first key word, the high half the second; the counter is word 0
    assert uniform24((7 << 32) | 5, 9) == (philox4x32_10((9, 0, 0, 0), (5, 7))[0] >> 8) / 2 ** 24
    assert uniform24(5, 9) != uniform24(5 << 32, 9)
    rs = [uniform24(12345, c) for c in range(2000)]
    assert all(0.0 <= r < 1.0 for r in rs)
    assert abs(np.mean(rs) - 0.5) < 0.03 and len(set(rs)) == len(rs)


def test_draw_walks_ids_not_sorted_order():
    # p = (1/6, 2/6, 3/6): running sums in id order 1/6, 1/2, 1 (sorted order would be 1/2, 5/6, 1)
    lg = LN([1.0, 2.0, 3.0])
    assert sample_reference(lg, r=0.10)[0] == 0     # sorted order would give id 2
    assert sample_reference(lg, r=0.20)[0] == 1
    assert sample_reference(lg, r=0.45)[0] == 1
    assert sample_reference(lg, r=0.60)[0] == 2
    tok, lp, ids, probs = sample_reference(lg, r=0.6, display_k=3)
    assert list(ids) == [2, 1, 0]
    np.testing.assert_allclose(probs, [0.5, 1 / 3, 1 / 6], rtol=1e-6)
    assert lp == pytest.approx(math.log(0.5), rel=1e-6)


def test_top_k_keeps_sorted_prefix_and_renormalises():
    lg = LN([1.0, 2.0, 3.0])
    # top-2 keeps ids 2 and 1: q = (0, 0.4, 0.6), id-order sums 0, 0.4, 1
    _, q = filtered_probs(lg, top_k=2)
    np.testing.assert_allclose(q, [0.0, 0.4, 0.6], rtol=1e-6)
    assert sample_reference(lg, top_k=2, r=0.3)[0] == 1
    assert sample_reference(lg, top_k=2, r=0.5)[0] == 2
    rng = np.random.default_rng(0)
    x = rng.normal(size=1000).astype(np.float32)
    for r in (0.0, 0.3, 0.999):
        assert sample_reference(x, top_k=1, r=r)[0] == int(np.argmax(x))
    # top_k >= vocab and top_k <= 0 filter nothing
    np.testing.assert_array_equal(filtered_probs(x, top_k=1000)[1], filtered_probs(x, top_k=0)[1])


def test_top_p_cutoff():
    # p = (.1, .2, .3, .4): sorted sums .4, .7, .9, 1
    lg = LN([1.0, 2.0, 3.0, 4.0])
    _, q = filtered_probs(lg, top_p=0.35)           # first sum .4 >= .35: keep id 3
    np.testing.assert_array_equal(q, [0, 0, 0, 1])
    _, q = filtered_probs(lg, top_p=0.65)           # .7 >= .65: keep ids 3, 2
    np.testing.assert_allclose(q, [0, 0, 3 / 7, 4 / 7], rtol=1e-6)
    _, q = filtered_probs(lg, top_p=0.95)           # only the total reaches .95: keep all
    np.testing.assert_allclose(q, [0.1, 0.2, 0.3, 0.4], rtol=1e-6)
    # top-p scans only the top-k prefix: with k = 2 no prefix sum (.4, .7) reaches .8, keep both
    _, q = filtered_probs(lg, top_k=2, top_p=0.8)
    np.testing.assert_allclose(q, [0, 0, 3 / 7, 4 / 7], rtol=1e-6)
    x = np.random.default_rng(1).normal(size=500).astype(np.float32)
    assert sample_reference(x, top_p=1e-6, r=0.77)[0] == int(np.argmax(x))
    assert topp_margin(lg, top_p=0.65) == pytest.approx(0.05, abs=1e-6)


def test_temperature_closed_form():
    # T = 2 halves the logits: (0, 2 ln 2) -> (0, ln 2) -> p = (1/3, 2/3)
    lg = np.array([0.0, 2 * math.log(2.0)], np.float32)
    _, q = filtered_probs(lg, temperature=2.0)
    np.testing.assert_allclose(q, [1 / 3, 2 / 3], rtol=1e-6)
    # greedy reports softmax(logits / T) as well, and the argmax token
    tok, lp, ids, probs = sample_reference(lg, temperature=2.0, do_sample=False, display_k=2)
    assert tok == 1 and list(ids) == [1, 0]
    np.testing.assert_allclose(probs, [2 / 3, 1 / 3], rtol=1e-6)
    assert lp == pytest.approx(math.log(2 / 3), rel=1e-6)


def test_unfiltered_probs_match_scipy_softmax():
    x = (np.random.default_rng(2).normal(size=151936) * 3).astype(np.float32)
    for t in (1.0, 0.7, 1.6):
        _, q = filtered_probs(x, temperature=t)
        ref = softmax(x.astype(np.float64) / t)
        np.testing.assert_allclose(q, ref, rtol=2e-6, atol=1e-30)


def test_grid_of_r_reproduces_inverse_cdf_counts():
    # r = (i + 0.5) / N for i < N: id j is drawn about q_j * N times (exactly floor/ceil)
    lg = LN([3.0, 1.0, 0.5, 2.0, 1.5, 2.0]).astype(np.float32)
    for cfg in ({}, {"top_k": 4}, {"top_p": 0.6}, {"temperature": 0.5, "top_k": 3}):
        _, q = filtered_probs(lg, **cfg)
        N = 4000
        counts = np.bincount([sample_reference(lg, r=(i + 0.5) / N, **cfg)[0] for i in range(N)], minlength=6)
        assert np.all(np.abs(counts - q * N) <= 1.0), (cfg, counts, q * N)
        assert np.all(counts[q == 0] == 0)


def test_ties_keep_lower_ids_first():
    lg = np.array([1.0, 5.0, 5.0, 0.0, 5.0], np.float32)
    tok, _, ids, _ = sample_reference(lg, do_sample=False, display_k=5)
    assert tok == 1 and list(ids) == [1, 2, 4, 0, 3]
    _, q = filtered_probs(lg, top_k=2)               # the tie at the boundary keeps ids 1, 2 (not 4)
    assert q[1] > 0 and q[2] > 0 and q[4] == 0 and q[1] == q[2]
    # -0.0 and +0.0 compare equal: stable order by id either way round
    assert list(sample_reference(np.array([-0.0, 0.0], np.float32), do_sample=False, display_k=2)[2]) == [0, 1]
    assert list(sample_reference(np.array([0.0, -0.0], np.float32), do_sample=False, display_k=2)[2]) == [0, 1]


def test_fallback_and_logprob_floor():
    # r beyond the total mass: the last id with q > 0; nothing positive: id 0
    assert draw_from_probs(np.array([0.5, 0.25, 0.0, 0.0], np.float32), 0.9) == 1
    assert draw_from_probs(np.zeros(4, np.float32), 0.1) == 0
    # a token of probability 1 has log-probability log(1 + 1e-10)
    tok, lp, _, _ = sample_reference(np.array([0.0, 200.0], np.float32), r=0.5)
    assert tok == 1 and lp == pytest.approx(1e-10, abs=1e-15)
