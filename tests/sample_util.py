"""Float64 restatement of the sampler's definition for the sampling tests.

The reference's sampler (Gufo's sampling::SamplerState, called from
SelectNext, runner.cpp:300-325, with runner.cpp:31-35's defaults) is not
vendored, so its picks cannot be replayed; these helpers state the
definition the kernel and the oracle follow with numpy's own sort, softmax
and cumulative sum, and judge a pick by the interval its target falls in.
"""
import numpy as np


def penalized(x, penalty, ids):
    """Repetition penalty: l / p for l > 0, l * p otherwise, once per id."""
    x = np.asarray(x, np.float32).copy()
    if ids is None or penalty == 1.0:
        return x
    p = np.float32(penalty)
    hit = np.unique(np.asarray(ids, np.int64))
    hit = hit[(hit >= 0) & (hit < x.size)]
    x[hit] = np.where(x[hit] > 0, x[hit] / p, x[hit] * p)
    return x


def candidates(x, top_k):
    """Candidate order: descending logit, lower index first on ties; the
    whole vocabulary in index order when top_k is 0 or >= its size."""
    n = x.size
    if top_k == 0 or top_k >= n:
        return np.arange(n)
    return np.argsort(-x.astype(np.float64), kind="stable")[:top_k]


def probabilities(x, temperature, top_k, penalty=1.0, ids=None):
    """(candidate ids, float64 probabilities) of a row."""
    z = penalized(x, penalty, ids)
    order = candidates(z, top_k)
    w = np.exp((z[order].astype(np.float64) - z.max()) / temperature)
    return order, w / w.sum()


def consistent(x, temperature, top_k, penalty, ids, u, pick, rel=2e-5):
    """Whether `pick` is the inverse-CDF pick of uniform u, up to float
    rounding of the running sums (rel of the total at either edge)."""
    z = penalized(x, penalty, ids)
    if not temperature > 0 or top_k == 1:
        return pick == int(np.argmax(z))
    order, p = probabilities(x, temperature, top_k, penalty, ids)
    where = np.nonzero(order == pick)[0]
    if where.size != 1 or p[where[0]] == 0:
        return False
    j = where[0]
    cum = np.cumsum(p)
    lo = cum[j - 1] if j else 0.0
    return lo - rel <= u <= cum[j] + rel
