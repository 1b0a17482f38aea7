"""Pins the oracle's sampler against brute-force fp64 statements of the rules,
closed forms, invariants and the reference's own known-answer tests (CPU).

Reference anchors (paths under the reference repository):
  * CTRL repetition penalty over the set of history ids, divide positive /
    multiply non-positive: native-mac/Sources/TinyGPTApp/ModelController.swift:262-283
  * greedy argmax, lowest id on ties (strict '>'): wasm/src/model.cpp:489-493
  * top-k by value threshold: python_ref/model.py:219-222, ModelController.swift:292-302
  * byte-level masker KATs: native-mac/Tests/TinyGPTModelTests/ConstrainedGenTests.swift:228-270
  * sampling invariants: tests/test_phase1.py:169-186
Reported probabilities agree with fp64 softmax within 1e-5 relative, with no
absolute floor (they are float weights over the top-p mass, not the floored
integer masses the draw uses).  Kept sets and draws agree exactly except where
the fp64 prefix lies within 1e-6 of p or u (reported boundary cases).
"""
import numpy as np
import pytest

import bruteforce as bf

TOL_REL = 1e-5


def one_row(oracle, x, params, u, hist=None, mask_row=None, kept_cap=None):
    x = np.asarray(x, dtype=np.float32)[None, :]
    V = x.shape[1]
    table = None if mask_row is None else np.asarray(mask_row, dtype=np.uint32)[None, :]
    p = params.copy()
    if mask_row is not None:
        p["mask_state"] = 0
    h = None if hist is None else np.asarray(hist, dtype=np.int32)[None, :]
    r = oracle.sample_batch(x, p, np.float32([u]), hist=h, mask_table=table,
                            kept_cap=kept_cap or V, want_post=True)
    return r


def rand_params(oracle, g, V):
    return oracle.make_params(
        1,
        temperature=float(g.choice([0.0, 0.3, 0.7, 1.0, 1.7])),
        top_k=int(g.choice([0, 1, 2, 5, V // 3, V - 1, V, V + 5])),
        top_p=float(g.choice([1.0, 0.95, 0.5, 0.1, 0.999])),
        repetition=float(g.choice([1.0, 1.1, 1.3, 0.8])),
        presence=float(g.choice([0.0, 0.5, -0.4])),
        frequency=float(g.choice([0.0, 0.3])),
    )


@pytest.mark.parametrize("seed", range(40))
def test_matches_bruteforce(oracle, seed):
    g = np.random.default_rng(1000 + seed)
    V = int(g.choice([7, 64, 256, 300]))
    x = (g.standard_normal(V) * g.choice([0.5, 2.0, 3.0])).astype(np.float32)
    if seed % 4 == 0:  # exact ties (planted spikes)
        x[g.choice(V, size=min(8, V), replace=False)] = 4.0
    if seed % 5 == 1:  # coarse values: many ties everywhere
        x = np.round(x).astype(np.float32)
    hist = g.integers(-3, V + 3, size=int(g.integers(0, 40))).astype(np.int32)
    params = rand_params(oracle, g, V)
    mask_row = None
    if seed % 3 == 2:
        bits = g.random(V) < 0.4
        mask_row = np.zeros((V + 31) // 32, dtype=np.uint32)
        for v in np.nonzero(bits)[0]:
            mask_row[v >> 5] |= np.uint32(1) << np.uint32(v & 31)
    u = float(np.float32(g.integers(0, 1 << 24) / (1 << 24)))
    r = one_row(oracle, x, params, u, hist=hist, mask_row=mask_row)
    ref = bf.sample(x, hist, params[0], u, mask_row)
    # post-penalty / mask / temperature logits: same float32 values
    np.testing.assert_array_equal(r["post"][0], ref["y"])
    res = r["res"][0]
    if ref["greedy"] or len(ref["kept"]) == 0:
        assert res["token"] == ref["token"]
        return
    kk = len(ref["kept"])
    assert res["n_topk"] == kk
    np.testing.assert_array_equal(r["kept_ids"][0][:kk], ref["kept"])
    # probabilities of the top-p survivors vs fp64 softmax renormalised
    ntp = res["n_topp"]
    pr = ref["probs"][:ntp] / ref["probs"][:ntp].sum()
    got = r["kept_probs"][0][:ntp].astype(np.float64)
    assert np.all(np.abs(got - pr) <= TOL_REL * pr)
    if ref["topp_margin"] > 1e-6:
        assert ntp == ref["ntopp"]
        if ref["draw_margin"] > 1e-6:
            assert res["token"] == ref["token"]


def test_greedy_lowest_id_on_ties(oracle):
    # model.cpp:491-493: strict '>' keeps the first (lowest) id among equal maxima
    x = np.float32([1.0, 5.0, 2.0, 5.0, 5.0, -1.0])
    p = oracle.make_params(1, temperature=0.0)
    assert one_row(oracle, x, p, 0.0)["ids"][0] == 1
    x = np.float32([-np.inf, np.nan, 3.0, 3.0])
    assert one_row(oracle, x, p, 0.0)["ids"][0] == 2


def test_repetition_penalty_ctrl(oracle):
    # ModelController.swift:276-279: x > 0 -> x / r, else x * r, once per distinct id
    x = np.float32([2.0, -2.0, 0.0, 4.0, 1.0])
    hist = np.int32([0, 0, 0, 1, 2, 7, -1])  # ids 7, -1 out of range: ignored
    p = oracle.make_params(1, temperature=1.0, repetition=2.0)
    y = one_row(oracle, x, p, 0.5, hist=hist)["post"][0]
    np.testing.assert_array_equal(y, np.float32([1.0, -4.0, 0.0, 4.0, 1.0]))
    # for r > 1 a penalised logit never increases (positive ones shrink toward
    # zero, non-positive ones are multiplied by r), and repeats change nothing
    g = np.random.default_rng(7)
    x = g.standard_normal(50).astype(np.float32) * 3
    h1 = np.int32([3, 4, 5])
    h2 = np.int32([3, 3, 3, 4, 5, 5])
    p = oracle.make_params(1, temperature=1.0, repetition=1.3)
    y1 = one_row(oracle, x, p, 0.1, hist=h1)["post"][0]
    y2 = one_row(oracle, x, p, 0.1, hist=h2)["post"][0]
    np.testing.assert_array_equal(y1, y2)
    assert np.all(y1 <= x)
    pos = [i for i in (3, 4, 5) if x[i] > 0]
    assert np.all(np.abs(y1[pos]) < np.abs(x[pos]))
    assert np.all(y1[[i for i in range(50) if i not in (3, 4, 5)]] == x[[i for i in range(50) if i not in (3, 4, 5)]])


def test_presence_frequency_linear_in_counts(oracle):
    # OpenAI definition: x - c * freq - (c > 0) * presence (no reference counterpart)
    x = np.zeros(8, dtype=np.float32)
    hist = np.int32([1, 2, 2, 3, 3, 3])
    p = oracle.make_params(1, temperature=1.0, presence=0.5, frequency=0.25)
    y = one_row(oracle, x, p, 0.2, hist=hist)["post"][0]
    np.testing.assert_array_equal(y[:4], np.float32([0.0, -0.75, -1.0, -1.25]))
    assert np.all(y[4:] == 0.0)


def test_temperature_is_scaling(oracle):
    """y = x / T correctly rounded (Serve.swift:1499, wasm/src/model.cpp:499).
    The float64 quotient of two floats rounded to float32 is the correctly
    rounded float32 quotient (53 >= 2 * 24 + 2, so the double rounding is
    harmless); the rule z * (1 / T) fails this on about a quarter of ids."""
    g = np.random.default_rng(9)
    x = (g.standard_normal(4096) * 3).astype(np.float32)
    x[:4] = [0.0, -0.0, 1e-38, -7.5]
    for T in (0.3, 0.7, 1.0, 1.5, 2.3, 1e-4, 3e3):
        p = oracle.make_params(1, temperature=T)
        y = one_row(oracle, x, p, 0.5, kept_cap=1)["post"][0]
        exact = (x.astype(np.float64) / np.float64(np.float32(T))).astype(np.float32)
        np.testing.assert_array_equal(y.view(np.uint32), exact.view(np.uint32), err_msg=f"T={T}")


def _mask_from_ids(V, ids):
    m = np.zeros((V + 31) // 32, dtype=np.uint32)
    for v in ids:
        m[v >> 5] |= np.uint32(1) << np.uint32(v & 31)
    return m


def test_mask_kats_restated(oracle):
    # ConstrainedGenTests.swift:228-245: at the start of an object schema only '{' is
    # legal for a byte-level vocab.  As a table row: one bit, id 123.
    g = np.random.default_rng(11)
    V = 256
    row = _mask_from_ids(V, [ord("{")])
    for T in (0.0, 0.8):
        for s in range(5):
            x = (g.standard_normal(V) * 3).astype(np.float32)
            p = oracle.make_params(1, temperature=T, top_k=40, top_p=0.95)
            r = one_row(oracle, x, p, float(g.random(dtype=np.float32)), mask_row=row)
            assert r["ids"][0] == ord("{")
    # :247-258 a complete FSM without EOS masks everything: no token (-1)
    r = one_row(oracle, x, oracle.make_params(1, temperature=0.8), 0.3, mask_row=np.zeros(8, np.uint32))
    assert r["ids"][0] == -1
    # :260-269 complete FSM with EOS 42: only 42 is allowed
    r = one_row(oracle, x, oracle.make_params(1, temperature=0.8, top_k=5), 0.99,
                mask_row=_mask_from_ids(V, [42]))
    assert r["ids"][0] == 42


def test_full_mask_is_identity(oracle):
    g = np.random.default_rng(12)
    x = (g.standard_normal(300) * 2).astype(np.float32)
    p = oracle.make_params(1, temperature=0.9, top_k=20, top_p=0.9)
    full = np.full((300 + 31) // 32, 0xFFFFFFFF, dtype=np.uint32)
    a = one_row(oracle, x, p, 0.37)
    b = one_row(oracle, x, p, 0.37, mask_row=full)
    assert a["ids"][0] == b["ids"][0]
    np.testing.assert_array_equal(a["kept_ids"], b["kept_ids"])


@pytest.mark.parametrize("T,k", [(0.3, 1024), (0.25, 600), (1.0, 1999)])
def test_tiny_probabilities_relative(oracle, T, k):
    """Long tails (kept weights down to ~1e-30 at T=0.3, ~1e-9 at T=1, below
    the 2^-40 mass unit): every reported probability is within 1e-5 relative of the fp64
    softmax of the canonical logits over the top-p survivors."""
    g = np.random.default_rng(int(T * 100) + k)
    V = 2000
    x = (g.standard_normal(V) * 3.0).astype(np.float32)
    p = oracle.make_params(1, temperature=T, top_k=k, top_p=1.0)
    r = oracle.sample_batch(x[None], p, np.float32([0.5]), kept_cap=V, want_post=True)
    ntp = int(r["res"]["n_topp"][0])
    assert ntp == k
    y = r["post"][0][r["kept_ids"][0][:ntp]].astype(np.float64)
    e = np.exp(y - y.max())
    pr = e / e.sum()
    got = r["kept_probs"][0][:ntp].astype(np.float64)
    assert pr.min() < 1e-8  # the tail reaches below the 2^-40 mass resolution
    assert np.max(np.abs(got - pr) / pr) <= TOL_REL


def test_draw_is_inverse_cdf(oracle):
    """Sweeping u over a uniform grid visits each survivor with frequency equal
    to its probability (the draw is an inverse CDF), to within 2 grid steps."""
    g = np.random.default_rng(13)
    V = 200
    x = (g.standard_normal(V) * 1.5).astype(np.float32)
    p = oracle.make_params(1, temperature=0.9, top_k=30, top_p=0.9)
    N = 1 << 14
    u = ((np.arange(N) + 0.5) / N).astype(np.float32)
    r = oracle.sample_batch(np.repeat(x[None], N, 0), np.repeat(p, N), u, kept_cap=V)
    ids = r["ids"]
    ntp = r["res"]["n_topp"][0]
    kept = r["kept_ids"][0][:ntp]
    probs = r["kept_probs"][0][:ntp].astype(np.float64)
    counts = np.array([(ids == k).sum() for k in kept]) / N
    assert np.all(np.abs(counts - probs) <= 2.0 / N)
    assert set(np.unique(ids)) <= set(kept.tolist())
    # the draw walks survivors in order: ids are piecewise constant in u
    firsts = [np.argmax(ids == k) for k in kept if (ids == k).any()]
    assert firsts == sorted(firsts)


def test_invariants_test_phase1(oracle):
    # test_phase1.py:169-186: same seed -> same ids; different seeds differ;
    # greedy deterministic.  Here the seed is the host uniform stream.
    g = np.random.default_rng(14)
    V, steps = 256, 30
    x = (g.standard_normal((steps, V)) * 2).astype(np.float32)
    p = np.repeat(oracle.make_params(1, temperature=0.9, top_k=20), steps)

    def run(seed):
        gg = np.random.default_rng(seed)
        u = (gg.integers(0, 1 << 24, size=steps) / (1 << 24)).astype(np.float32)
        return oracle.sample_batch(x, p, u)["ids"].tolist()

    assert run(123) == run(123)
    assert run(123) != run(456)
    pg = np.repeat(oracle.make_params(1, temperature=0.0), steps)
    a = oracle.sample_batch(x, pg, np.zeros(steps, np.float32))["ids"]
    b = oracle.sample_batch(x, pg, np.full(steps, 0.7, np.float32))["ids"]
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a, np.argmax(x, axis=1))


def test_reference_tie_rule_difference_is_counted(oracle):
    # python_ref/model.py:222 keeps every id tied with the k-th value; the
    # contract keeps exactly k (lowest ids first) and reports the difference.
    x = np.float32([5, 4, 4, 4, 4, 1, 0, 0])
    p = oracle.make_params(1, temperature=1.0, top_k=3)
    r = one_row(oracle, x, p, 0.5)
    assert r["res"]["n_topk"][0] == 3
    np.testing.assert_array_equal(r["kept_ids"][0][:3], [0, 1, 2])
    assert r["res"]["ref_tie_extra"][0] == 2


def test_invalid_rows(oracle):
    x = np.zeros(16, dtype=np.float32)
    bad = [
        dict(temperature=float("nan")),
        dict(temperature=float("inf")),
        dict(temperature=1e-45),
        dict(temperature=1.0, top_p=0.0),
        dict(temperature=1.0, top_p=float("nan")),
        dict(temperature=1.0, repetition=0.0),
        dict(temperature=1.0, presence=float("inf")),
    ]
    for kw in bad:
        r = one_row(oracle, x, oracle.make_params(1, **kw), 0.5)
        assert r["ids"][0] == -2, kw
    for u in (1.0, -0.1, float("nan")):
        assert one_row(oracle, x, oracle.make_params(1, temperature=1.0), u)["ids"][0] == -2
    # greedy rows ignore u and top_p
    assert one_row(oracle, x, oracle.make_params(1, temperature=0.0, top_p=0.0), 5.0)["ids"][0] == 0


def test_boundary_uniforms(oracle):
    g = np.random.default_rng(15)
    x = (g.standard_normal(1000) * 3).astype(np.float32)
    p = oracle.make_params(1, temperature=0.8, top_k=50, top_p=0.9)
    r0 = one_row(oracle, x, p, 0.0, kept_cap=50)
    assert r0["ids"][0] == r0["kept_ids"][0][0]  # u = 0 picks the most likely id
    r1 = one_row(oracle, x, p, float(np.float32(1 - 2.0**-24)), kept_cap=50)
    assert r1["ids"][0] == r1["kept_ids"][0][r1["res"]["n_topp"][0] - 1]
