"""Brute-force fp64 statements of the sampling rules, used to pin the oracle.

Written independently of oracle/tgs_oracle.c: penalties and temperature are
evaluated with numpy float32 element-wise operations, the order is a full
lexicographic sort, probabilities are fp64 softmax values and the top-p cut
and the draw are fp64 prefix sums.  Only small rows are meant to go through
here.
"""
from __future__ import annotations

import numpy as np


def post_logits(x, hist, params, mask_row=None):
    """Canonical post-penalty / mask / temperature logits (float32, -inf where
    not allowed).  Returns (y, greedy)."""
    x = np.asarray(x, dtype=np.float32)
    V = x.size
    T = np.float32(params["temperature"])
    greedy = bool(params["flags"] & 1) or T <= 0
    z = x.copy()
    rep = np.float32(params["repetition"])
    pres = np.float32(params["presence"])
    freq = np.float32(params["frequency"])
    neutral = rep == 1 and pres == 0 and freq == 0
    if hist is not None and len(hist) and not neutral:
        h = np.asarray(hist)
        h = h[(h >= 0) & (h < V)]
        cnt = np.bincount(h, minlength=V)
        ids = np.nonzero(cnt)[0]
        zi = z[ids]
        if rep != 1:
            zi = np.where(zi > 0, zi / rep, zi * rep).astype(np.float32)
        zi = (zi - freq * cnt[ids].astype(np.float32)).astype(np.float32)
        zi = (zi - pres).astype(np.float32)
        z[ids] = zi
    y = z if greedy else (z / T).astype(np.float32)  # IEEE float32 division (Serve.swift:1499)
    allowed = y > -np.inf  # False for NaN
    if mask_row is not None:
        bits = (np.asarray(mask_row, dtype=np.uint32)[np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1
        allowed &= bits.astype(bool)
    y = np.where(allowed, y, np.float32(-np.inf)).astype(np.float32)
    return y, greedy


def order(y):
    """Allowed ids sorted by (y desc, id asc)."""
    ids = np.nonzero(y > -np.inf)[0]
    o = np.lexsort((ids, -y[ids].astype(np.float64)))
    return ids[o]


def sample(x, hist, params, u, mask_row=None):
    """Returns dict(token, kept (top-k ids), probs (fp64 over the top-k set),
    ntopp, topp_margin, draw_margin) in fp64 arithmetic."""
    y, greedy = post_logits(x, hist, params, mask_row)
    ids = order(y)
    if len(ids) == 0:
        return dict(token=-1, kept=ids, probs=np.zeros(0), ntopp=0, y=y, greedy=greedy,
                    topp_margin=np.inf, draw_margin=np.inf)
    if greedy:
        return dict(token=int(ids[0]), kept=ids[:1], probs=np.ones(1), ntopp=1, y=y, greedy=True,
                    topp_margin=np.inf, draw_margin=np.inf)
    V = y.size
    k = int(params["top_k"])
    kk = min(k, len(ids)) if 1 <= k < V else len(ids)
    kept = ids[:kk]
    yk = y[kept].astype(np.float64)
    e = np.exp(yk - yk[0])
    p = e / e.sum()
    c = np.cumsum(p)
    top_p = float(params["top_p"])
    ntopp = kk
    topp_margin = np.inf
    if top_p < 1:
        ntopp = int(np.searchsorted(c, top_p - 1e-15, side="left")) + 1
        ntopp = min(ntopp, kk)
        topp_margin = float(np.min(np.abs(c[max(0, ntopp - 2):ntopp] - top_p)))
    cp = c[:ntopp] / c[ntopp - 1]
    pick = int(np.searchsorted(cp, float(u), side="right"))
    pick = min(pick, ntopp - 1)
    draw_margin = float(np.min(np.abs(np.concatenate([[0.0], cp]) - float(u))))
    return dict(token=int(kept[pick]), kept=kept, probs=p, ntopp=ntopp, y=y, greedy=False,
                topp_margin=topp_margin, draw_margin=draw_margin)
