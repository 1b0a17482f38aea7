"""The float64 restatement of teacher-forced token log-probabilities
(oracle.token_logprobs, Serve.swift:983-993) pinned by closed forms and a
library routine.  CPU only."""
import numpy as np
import pytest


def test_uniform_row_gives_minus_log_v(oracle):
    for V in (1, 7, 4096, 128256):
        lp, lse = oracle.token_logprobs(np.full((1, V), 0.3, np.float32), [V - 1])
        assert lp[0] == pytest.approx(-np.log(V), abs=1e-12)
        assert lse[0] == pytest.approx(float(np.float32(0.3)) + np.log(V), abs=1e-12)


def test_two_valued_row_closed_form(oracle):
    # one id at a, n - 1 ids at c: p(a) = 1 / (1 + (n - 1) e^(c - a))
    n, a, c = 1000, 5.0, 1.0
    x = np.full((2, n), c, np.float32)
    x[:, 17] = a
    lp, _ = oracle.token_logprobs(x, [17, 3])
    assert lp[0] == pytest.approx(-np.log1p((n - 1) * np.exp(c - a)), abs=1e-12)
    assert lp[1] == pytest.approx((c - a) - np.log1p((n - 1) * np.exp(c - a)), abs=1e-12)


def test_shift_invariance_and_library_logsumexp(oracle):
    from scipy.special import logsumexp

    g = np.random.default_rng(3)
    # multiples of 2^-10 in (-16, 16): adding 16 is exact in float32
    x = (np.round(np.clip(g.normal(0.0, 3.0, (5, 3001)), -15.9, 15.9) * 1024) / 1024).astype(np.float32)
    tok = g.integers(0, 3001, 5)
    lp, lse = oracle.token_logprobs(x, tok)
    lp2, _ = oracle.token_logprobs(x + np.float32(16.0), tok)
    np.testing.assert_allclose(lp, lp2, atol=1e-9)
    ref = logsumexp(x.astype(np.float64), axis=1)
    np.testing.assert_allclose(lse, ref, rtol=0, atol=1e-10)
    np.testing.assert_allclose(lp, x[np.arange(5), tok].astype(np.float64) - ref, atol=1e-10)
    assert np.all(lp < 0)


def test_special_values(oracle):
    x = np.zeros((6, 8), np.float32)
    x[1, 2] = -np.inf  # -inf adds nothing
    x[2, :] = -np.inf  # only -inf: NaN
    x[3, 5] = np.nan
    x[4, 0] = np.inf
    lp, lse = oracle.token_logprobs(x, [0, 3, 0, 0, 0, 8])
    assert lp[0] == pytest.approx(-np.log(8))
    assert lp[1] == pytest.approx(-np.log(7))
    assert np.isnan(lp[2:]).all() and np.isnan(lse[2:5]).all()
    assert lse[5] == pytest.approx(np.log(8))  # token outside [0, V): NaN logprob, finite lse


def test_bf16_rows_and_strided_columns(oracle):
    from tinygpt_amd import workloads as W

    g = np.random.default_rng(4)
    x = g.normal(0.0, 2.0, (3, 40)).astype(np.float32)
    xb = W.f32_to_bf16_bits(x)
    up = (xb.astype(np.uint32) << np.uint32(16)).view(np.float32)
    lp, _ = oracle.token_logprobs(xb, [1, 2, 3], V=33)
    lp2, _ = oracle.token_logprobs(up[:, :33], [1, 2, 3])
    np.testing.assert_array_equal(lp, lp2)
