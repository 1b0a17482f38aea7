"""Chi-square agreement of a draw histogram with a probability vector (used
by the comparisons against the reference's C++ sampler fixtures)."""
from __future__ import annotations

import numpy as np
from scipy.stats import chi2

ALPHA = 1e-6


def agrees(counts, prob, alpha=ALPHA):
    """(statistic, threshold, support ok) of histogram `counts` against
    probabilities `prob`; bins expecting fewer than 5 draws are pooled.
    `support ok` is False when a drawn id has probability 0."""
    counts = np.asarray(counts)
    prob = np.asarray(prob, dtype=np.float64)
    n = counts.sum()
    e = prob * n
    support_ok = bool(np.all(prob[counts > 0] > 0))
    big = e >= 5
    obs = np.array(list(counts[big]) + [counts[~big].sum()], float)
    exp = np.array(list(e[big]) + [e[~big].sum()], float)
    if exp[-1] == 0:
        obs, exp = obs[:-1], exp[:-1]
    stat = float(np.sum((obs - exp) ** 2 / np.maximum(exp, 1e-300)))
    thr = float(chi2.isf(alpha, max(1, len(obs) - 1)))
    return stat, thr, support_ok
