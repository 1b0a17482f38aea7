"""The oracle against the reference's own C++ sampler (tg_generate,
wasm/src/model.cpp:473-519), through the fixtures tests/golden/make_tg_ref.py
wrote from oracle/_ref (the reference sources compiled where they lie).

tg_generate draws with its own mt19937 stream and walks the CDF in id order,
while the canonical contract draws from a host uniform in (logit desc, id
asc) order; single draws therefore differ by design, and the comparison is:
  - greedy decoding: the same ids, step by step (exact);
  - sampling: the reference's draw histogram over 20000 seeds against the
    oracle's probabilities (chi-square, significance 1e-6), and every id the
    reference drew is in the oracle's kept set.
Plausible mistakes (temperature applied as a product or not at all, top-k
off by one or ignored), planted through the oracle's parameters, must be
rejected by at least one case, which shows the comparison has the power to
see them.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import pyoracle
from refstats import agrees

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "tg_ref_c1.npz")
REF_LIB = os.path.join(os.path.dirname(HERE), "oracle", "_ref", "libtg_ref.so")


@pytest.fixture(scope="module")
def fx():
    return dict(np.load(FIX, allow_pickle=False))


def oracle_probs(logits, T, k):
    """Oracle kept set and normalised probabilities for one row (top-p off)."""
    V = logits.size
    p = pyoracle.make_params(1, temperature=T, top_k=k)
    r = pyoracle.sample_batch(logits[None, :].astype(np.float32), p, np.zeros(1, np.float32),
                              kept_cap=V)
    ids = r["kept_ids"][0]
    keep = ids >= 0
    prob = np.zeros(V)
    prob[ids[keep]] = r["kept_probs"][0][keep]
    return prob


def test_greedy_continuation_matches_reference(fx):
    logits = fx["greedy_logits"]
    n = logits.shape[0]
    p = pyoracle.make_params(n, temperature=0.0)
    got = pyoracle.sample_batch(logits, p, np.zeros(n, np.float32))["ids"]
    np.testing.assert_array_equal(got, fx["greedy_out"])


@pytest.mark.parametrize("case", range(4))
def test_sampling_distribution_matches_reference(fx, case):
    prob = oracle_probs(fx["samp_logits"][case], float(fx["samp_T"][case]), int(fx["samp_k"][case]))
    stat, thr, support_ok = agrees(fx["samp_counts"][case], prob)
    assert support_ok, "the reference drew an id outside the oracle's kept set"
    assert stat < thr, f"chi-square {stat:.1f} >= {thr:.1f}"
    k = int(fx["samp_k"][case])
    if k:
        assert np.count_nonzero(prob) == k


MISTAKES = {
    "temperature multiplied": lambda T, k: (1.0 / T, k),
    "temperature ignored": lambda T, k: (1.0, k),
    "top-k one too many": lambda T, k: (T, k + 1 if k else k),
    "top-k one too few": lambda T, k: (T, k - 1 if k > 1 else k),
    "top-k ignored": lambda T, k: (T, 0),
}


@pytest.mark.parametrize("name", sorted(MISTAKES))
def test_planted_mistakes_are_rejected(fx, name):
    rejected = []
    for case in range(len(fx["samp_T"])):
        T, k = float(fx["samp_T"][case]), int(fx["samp_k"][case])
        T2, k2 = MISTAKES[name](T, k)
        if (T2, k2) == (T, k):
            continue
        stat, thr, support_ok = agrees(fx["samp_counts"][case], oracle_probs(fx["samp_logits"][case], T2, k2))
        rejected.append(not support_ok or stat >= thr)
    assert rejected and any(rejected), f"planted mistake '{name}' was not detected"


def test_fixture_is_current_with_reference_build(fx):
    """Where oracle/_ref is built, its greedy decode still gives the fixture."""
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_tg_ref", os.path.join(HERE, "golden", "make_tg_ref.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    L = mk.load()
    m = mk.trained_model(L)
    try:
        g = mk.generate(L, m, mk.GREEDY_PROMPT, mk.GREEDY_NEW, 0.0, 0, 0)
        np.testing.assert_array_equal(g, fx["greedy_out"])
        row = mk.last_logits(L, m, list(mk.GREEDY_PROMPT))
        np.testing.assert_array_equal(row, fx["greedy_logits"][0])
    finally:
        L.tg_model_free(m)
