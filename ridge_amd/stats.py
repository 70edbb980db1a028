"""Statistics of the accuracy report and the pruner, from their definitions.

- Mid-ranks: the values of a sample are ordered; a run of equal values occupies
  a block of consecutive positions and each of them is given the mean position
  of the block (positions counted from 1).
- Spearman's rho: Pearson's product-moment correlation of the two mid-rank
  vectors. It is undefined when either side has no variance (every config of a
  shape predicted alike), and is then reported as nan rather than 0.
- Quantiles: numpy's linear interpolation between order statistics.
- Regret of a pick: (best measured - measured of the pick) / best measured.
- Expected regret of a uniformly random shortlist of k of n configs: with the
  measured values sorted best first, m_1 >= ... >= m_n, the best of the
  shortlist is m_i exactly when it holds config i and none of the i - 1 better
  ones, which C(n - i, k - 1) of the C(n, k) shortlists do.
"""

import bisect
import math
import statistics

import numpy as np

NAN = float("nan")


def midranks(xs):
    """Rank of every element of `xs` (1-based), ties sharing their mean position."""
    ordered = sorted(xs)
    out = []
    for x in xs:
        below = bisect.bisect_left(ordered, x)
        equal = bisect.bisect_right(ordered, x) - below
        out.append(below + (equal + 1) / 2.0)
    return out


def pearson(a, b):
    """Product-moment correlation; nan for fewer than two pairs or a constant side."""
    if len(a) != len(b):
        raise ValueError("correlation of samples of different sizes (%d, %d)" % (len(a), len(b)))
    if len(a) < 2:
        return NAN
    try:
        return statistics.correlation(list(map(float, a)), list(map(float, b)))
    except statistics.StatisticsError:  # one side has no variance
        return NAN


def spearman(a, b):
    return pearson(midranks(a), midranks(b))


def quantile(xs, pct):
    """The pct-th percentile (0..100); nan for an empty sample."""
    return float(np.percentile(np.asarray(xs, dtype=float), pct)) if len(xs) else NAN


def regret(best, picked):
    return (best - picked) / best


def expected_random_regret(measured, k):
    """Exact expected regret of the best of a uniformly random k-subset."""
    n = len(measured)
    if not 1 <= k <= n:
        raise ValueError("shortlist of %d from %d configs" % (k, n))
    ranked = sorted(measured, reverse=True)
    best = ranked[0]
    total = math.comb(n, k)
    return sum(math.comb(n - i, k - 1) * regret(best, m) for i, m in enumerate(ranked, start=1)) / total


def top_tie(pred, meas):
    """The measured values of the configs tied at the top of the prediction."""
    top = max(pred)
    return [m for p, m in zip(pred, meas) if p == top]


def best_rank_range(pred, meas):
    """(optimistic, pessimistic) 1-based position of the measured-best config in
    the predicted order, over every order of the configs it ties with."""
    p_best = pred[max(range(len(meas)), key=lambda i: meas[i])]
    above = sum(p > p_best for p in pred)
    level = sum(p == p_best for p in pred)
    return above + 1, above + level
