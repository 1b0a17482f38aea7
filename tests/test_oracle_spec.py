"""Pins the oracle's speculative verification (CPU).

Reference: native-mac/Sources/TinyGPT/SpeculativeDecode.swift:121-210
(stochastic: accept iff u < p_target/p_draft, residual max(p_t - p_d, 0),
bonus token from the next target row) and :41-98 (greedy).
  * the canonical softmax denominator matches fp64 within 1e-6 relative;
  * accept/reject decisions match an fp64 evaluation except within 1e-6;
  * Leviathan et al. Thm 3.5: the first emitted token is distributed as
    softmax(target) whatever the draft (Monte Carlo at V = 8).
"""
import numpy as np
import pytest


def softmax64(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def test_row_stats_match_fp64(oracle):
    g = np.random.default_rng(21)
    for V in (5, 1000, 1024, 1025, 5000, 128256):
        y = (g.standard_normal(V) * 3).astype(np.float32)
        m, S = oracle.spec_row_stats(y)
        assert m == y.max()
        ref = np.exp(y.astype(np.float64) - float(m)).sum()
        assert abs(S - ref) <= 1e-6 * ref


@pytest.mark.parametrize("seed", range(6))
def test_accept_decisions_match_fp64(oracle, seed):
    g = np.random.default_rng(30 + seed)
    B, k, V = 16, 4, 300
    target = (g.standard_normal((B, k + 1, V)) * 2).astype(np.float32)
    draft = (target[:, :k] + g.standard_normal((B, k, V))).astype(np.float32)
    dtok = g.integers(0, V, size=(B, k)).astype(np.int32)
    T = np.float32(g.choice([0.5, 1.0, 1.3]))
    u_acc = (g.integers(0, 1 << 24, size=(B, k)) / (1 << 24)).astype(np.float32)
    u_res = (g.integers(0, 1 << 24, size=B) / (1 << 24)).astype(np.float32)
    r = oracle.spec_verify_batch(target, draft, dtok, np.full(B, T), u_acc, u_res)
    for b in range(B):
        n = r["n_acc"][b]
        assert 0 <= n <= k
        for j in range(n + (1 if n < k else 0)):
            pt = softmax64(target[b, j] / T)[dtok[b, j]]
            pd = softmax64(draft[b, j] / T)[dtok[b, j]]
            ratio = pt / max(pd, 1e-10)
            if abs(u_acc[b, j] - ratio) <= 1e-5 * max(1.0, ratio):
                break  # boundary case: either decision is allowed
            accepted = j < n
            assert accepted == (u_acc[b, j] < ratio), (b, j, u_acc[b, j], ratio)
        np.testing.assert_array_equal(r["out"][b, :n], dtok[b, :n])
        assert 0 <= r["out"][b, n] < V
        assert np.all(r["out"][b, n + 1:] == -1)


def test_greedy_verify(oracle):
    g = np.random.default_rng(40)
    B, k, V = 8, 5, 64
    target = g.standard_normal((B, k + 1, V)).astype(np.float32)
    am = target.argmax(-1)
    dtok = am[:, :k].copy().astype(np.int32)
    # sequence b mismatches at position b (b < k); the last ones accept all
    for b in range(min(B, k)):
        dtok[b, b] = (am[b, b] + 1) % V
    r = oracle.spec_verify_batch(target, target[:, :k].copy(), dtok, np.zeros(B), np.zeros((B, k)), np.zeros(B))
    for b in range(B):
        n = b if b < k else k
        assert r["n_acc"][b] == n
        np.testing.assert_array_equal(r["out"][b, :n], am[b, :n])
        assert r["out"][b, n] == am[b, n]


def test_leviathan_distribution(oracle):
    g = np.random.default_rng(41)
    V, N = 8, 200000
    t = (g.standard_normal(V) * 1.5).astype(np.float32)
    d = (g.standard_normal(V) * 1.5).astype(np.float32)
    pd = softmax64(d)
    pt = softmax64(t)
    cd = np.cumsum(pd)
    dtok = np.minimum(np.searchsorted(cd, g.random(N), side="right"), V - 1).astype(np.int32)
    target = np.broadcast_to(np.stack([t, t])[None], (N, 2, V)).copy()
    draft = np.broadcast_to(d[None, None], (N, 1, V)).copy()
    u_acc = (g.integers(0, 1 << 24, size=(N, 1)) / (1 << 24)).astype(np.float32)
    u_res = (g.integers(0, 1 << 24, size=N) / (1 << 24)).astype(np.float32)
    r = oracle.spec_verify_batch(target, draft, dtok[:, None], np.ones(N, np.float32), u_acc, u_res, nthreads=8)
    first = r["out"][:, 0]
    freq = np.bincount(first, minlength=V) / N
    sigma = np.sqrt(pt * (1 - pt) / N)
    assert np.all(np.abs(freq - pt) <= 5 * sigma + 1e-4), (freq, pt)
    # and the acceptance rate is sum(min(p_t, p_d))
    acc = (r["n_acc"] == 1).mean()
    assert abs(acc - np.minimum(pt, pd).sum()) <= 5 * np.sqrt(0.25 / N)


def test_invalid_inputs(oracle):
    V, k = 16, 2
    target = np.zeros((1, k + 1, V), np.float32)
    draft = np.zeros((1, k, V), np.float32)
    for dt, T, ua in [([[0, V]], 1.0, [[0.1, 0.1]]), ([[0, 1]], float("nan"), [[0.1, 0.1]]),
                      ([[0, 1]], 1.0, [[1.0, 0.1]])]:
        r = oracle.spec_verify_batch(target, draft, np.int32(dt), np.float32([T]), np.float32(ua), np.float32([0.5]))
        assert r["out"][0, 0] == -2 and r["n_acc"][0] == -1
