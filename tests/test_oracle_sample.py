"""Pins the oracle's sampler (orc_sample) before the kernel is checked
against it.

The reference's sampler is Gufo's host sampler, which the reference does not
carry (SelectNext, runner.cpp:300-325), so there are no golden picks: parity
with it stays unpinned. What pins the restatement instead:
  * the greedy cases reduce to std::max_element (tests/session_test.cpp:
    32-34), ties to the first index;
  * frequencies: a grid of uniforms through the inverse CDF must hit every
    candidate in proportion to numpy's float64 softmax over numpy's sort;
  * closed forms of the penalty (a penalized leader loses to the runner-up;
    a negative logit moves away from zero) and of top-k ties (the lower
    index is kept).
"""
import numpy as np
import pytest

import oracle as O
from sample_util import consistent, probabilities


def row(seed, n, scale=3.0):
    return (scale * np.random.default_rng(seed).standard_normal(n)).astype(np.float32)


def test_greedy_cases_are_max_element():
    x = row(1, 5000)
    x[17] = x[4000] = x.max() + 1.0
    for t, k in [(0.0, 50), (-1.0, 0), (0.7, 1), (float("-inf"), 3)]:
        assert O.sample(x, t, k) == 17
    assert O.sample(np.full(64, -2.0, np.float32), 0.0, 0) == 0


@pytest.mark.parametrize("t,k", [(0.7, 5), (1.0, 0), (0.1, 50), (2.0, 20)])
def test_inverse_cdf_frequencies(t, k):
    n, grid = 40, 20000
    x = row(2 + k, n, 1.5)
    order, p = probabilities(x, t, k)
    counts = np.zeros(n, np.int64)
    for i in range(grid):
        counts[O.sample(x, t, k, u=(i + 0.5) / grid)] += 1
    want = np.zeros(n)
    want[order] = p * grid
    # each candidate's share of the grid is exact up to the two edge cells
    assert np.max(np.abs(counts - want)) <= 2.0
    assert counts[np.setdiff1d(np.arange(n), order)].sum() == 0


def test_picks_follow_the_cumulative_definition():
    rng = np.random.default_rng(3)
    for case in range(200):
        n = int(rng.integers(2, 3000))
        x = row(100 + case, n, float(rng.uniform(0.5, 8)))
        t = float(rng.choice([0.1, 0.5, 1.0, 3.0]))
        k = int(rng.choice([0, 2, 5, 50, 1024, n]))
        pen = rng.integers(0, n + 10, size=int(rng.integers(0, 64))).astype(np.uint32)
        u = float(rng.random())
        pick = O.sample(x, t, k, 1.1, pen, u)
        assert consistent(x, t, k, 1.1, pen, u, pick), (case, n, t, k, u, pick)


def test_penalty_closed_form():
    x = np.array([0.5, 2.0, 1.9, -1.0, -1.05], np.float32)
    assert O.sample(x, 0.0, 0) == 1
    assert O.sample(x, 0.0, 0, 1.1, [1]) == 2          # 2.0 / 1.1 < 1.9
    z = np.array([2.0, 1.7], np.float32)
    assert O.sample(z, 0.0, 0, 1.1, [0, 0, 0]) == 0    # 1.818 once, not 1.50 thrice
    assert O.sample(x, 0.0, 0, 1.1, [1, 99]) == 2      # ids past the row are padding
    y = np.array([-1.0, -1.05], np.float32)
    assert O.sample(y, 0.0, 0, 1.1, [0]) == 1          # -1.1 < -1.05


def test_topk_ties_keep_the_lower_index():
    x = np.array([3.0, 1.0, 1.0, 1.0, 0.0], np.float32)
    seen = {O.sample(x, 1.0, 2, u=(i + 0.5) / 1000) for i in range(1000)}
    assert seen == {0, 1}
