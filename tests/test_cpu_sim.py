"""The product HIP kernels, compiled for the host against the CPU simulation
in tests/cpu_sim (one OS thread per GPU thread, 64-lane waves, LDS poisoned
at every workgroup start) under AddressSanitizer and UBSan, checked against
the oracle.  Every memory access of the kernels on these batches is bounds
checked; a sanitizer report fails the test.  CPU only."""
import os
import shutil
import sys

import numpy as np
import pytest

import gpu_harness as H

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "cpu_sim"))

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


@pytest.fixture(scope="module")
def sim():
    import sim as S

    S.build()
    return S


def _batch(seed, B, V, oracle):
    from test_gpu_sampler import _random_batch

    return _random_batch(np.random.default_rng(seed), B, V, oracle)


def _check(sim, oracle, x, params, u, hist, hist_len, mask=None, hint=None, split=None, kept_cap=1025,
           noalloc=False):
    r = sim.run_sample(x, params, u, hist, hist_len, mask_table=mask, kept_cap=kept_cap, hint=hint, split=split,
                       noalloc=noalloc)
    o = oracle.sample_batch(x, params, u, hist=hist, hist_len=hist_len, mask_table=mask, kept_cap=kept_cap,
                            want_post=True)
    return r, o, H.compare(r, o, params, x.shape[1], what="sim")


def test_general_and_full_kernels(sim, oracle):
    x, params, u, hist, hist_len = _batch(11, 16, 256, oracle)
    _check(sim, oracle, x, params, u, hist, hist_len)


def test_gpu_skipped_batch_v256(sim, oracle):
    """The exact batch of the GPU test test_random_rows[256] (rng 500 + 256,
    B=64, history 64, no hint: chunk, merge, full-path and top-p kernels),
    which is skipped on the GPU because an earlier kernel layout faulted on
    it.  Every access of the current kernels on it is bounds checked here."""
    from test_gpu_sampler import _random_batch

    x, params, u, hist, hist_len = _random_batch(np.random.default_rng(500 + 256), 64, 256, oracle)
    r, _, _ = _check(sim, oracle, x, params, u, hist, hist_len)
    assert len(r["launches"]) >= 3  # chunk, full and top-p kernels all ran


def test_fast_kernel_with_hint(sim, oracle):
    import tinygpt_amd as tg

    x, params, u, hist, hist_len = _batch(12, 12, 300, oracle)
    params["top_k"] = np.random.default_rng(1).choice([1, 2, 5, 40, 63, 64], size=12)
    _check(sim, oracle, x, params, u, hist, hist_len, hint=tg.batch_hint(params, 300))


def test_split_rows_and_merge(sim, oracle):
    x, params, u, hist, hist_len = _batch(13, 4, 5000, oracle)
    _check(sim, oracle, x, params, u, hist, hist_len, split=3)


def test_grammar_mask(sim, oracle):
    V = 300
    g = np.random.default_rng(14)
    x, params, u, hist, hist_len = _batch(14, 8, V, oracle)
    table = g.integers(0, 1 << 32, size=(4, (V + 31) // 32), dtype=np.uint64).astype(np.uint32)
    table[1] = 0
    table[2, 0] = 1
    params["mask_state"] = np.array([0, 1, 2, 3, -1, 4, 0, 3])  # 4: out of range, id -2
    _check(sim, oracle, x, params, u, hist, hist_len, mask=table)


def test_bf16_rows(sim, oracle):
    from tinygpt_amd import workloads as W

    x, params, u, hist, hist_len = _batch(15, 8, 1000, oracle)
    xb = W.f32_to_bf16_bits(x)
    _check(sim, oracle, xb, params, u, hist, hist_len)


def test_rows_outside_the_hint_get_minus_3(sim, oracle):
    g = np.random.default_rng(55)
    B, V = 8, 3000
    x = g.standard_normal((B, V)).astype(np.float32)
    params = oracle.make_params(B, temperature=0.9, top_k=10, top_p=0.9)
    params["top_k"][3] = 50    # above the hint, fast kernel
    params["top_k"][5] = 0     # no usable top-k: full path not launched
    params["temperature"][6] = 0.0  # greedy: served under any hint
    u = np.full(B, 0.3, np.float32)
    o = oracle.sample_batch(x, params, u)
    for hint in (10, 200):
        r = sim.run_sample(x, params, u, hint=hint, post=False)
        expect = o["ids"].copy()
        expect[5] = -3
        if hint < 50:
            expect[3] = -3
        np.testing.assert_array_equal(r["ids"], expect)


def _k64_params(g, params, V):
    ks = np.array([1, 2, 5, 40, 63, 64])
    params["top_k"] = g.choice(ks[ks < V], size=params.size)
    return params


@pytest.mark.parametrize("split", [1, 2])
def test_k64_multi_tile_chunks(sim, oracle, split):
    """Fused top_k <= 64 kernel with chunks of several 8192-id tiles: later
    tiles of ascending rows overflow the candidate buffer (exact fallback)."""
    import tinygpt_amd as tg

    g = np.random.default_rng(40 + split)
    V = 20000
    x, params, u, hist, hist_len = _batch(40 + split, 7, V, oracle)
    params = _k64_params(g, params, V)
    _check(sim, oracle, x, params, u, hist, hist_len, hint=tg.batch_hint(params, V), split=split, kept_cap=64)


def test_k64_split_merge_16(sim, oracle):
    """Sixteen chunks per row: the last workgroup merges sixteen lists."""
    import tinygpt_amd as tg

    g = np.random.default_rng(44)
    V = 20000
    x, params, u, hist, hist_len = _batch(44, 7, V, oracle)
    params = _k64_params(g, params, V)
    _check(sim, oracle, x, params, u, hist, hist_len, hint=tg.batch_hint(params, V), split=16, kept_cap=64)


@pytest.mark.parametrize("path", ["k64", "general"])
def test_noalloc_entry_point(sim, oracle, path):
    """tgs_sample_noalloc: the same kernels on the static workspace (k64
    lists and counters as the first call on a device leaves them; the
    general path's chunk lists) and a mask table passed by pointer."""
    import tinygpt_amd as tg

    g = np.random.default_rng(46)
    V = 20000
    x, params, u, hist, hist_len = _batch(46, 7, V, oracle)
    mask = g.integers(0, 1 << 32, size=(3, (V + 31) // 32), dtype=np.uint64).astype(np.uint32)
    params["mask_state"] = g.integers(-1, 3, size=7)
    if path == "k64":
        params = _k64_params(g, params, V)
        _check(sim, oracle, x, params, u, hist, hist_len, mask=mask, hint=tg.batch_hint(params, V), split=4,
               kept_cap=64, noalloc=True)
    else:
        _check(sim, oracle, x, params, u, hist, hist_len, mask=mask, split=2, noalloc=True)


@pytest.mark.parametrize("split", [1, 3])
def test_k64_history_at_top(sim, oracle, split):
    """Rows whose largest logits are penalised history ids, small top_k: the
    chunk bounds come from the other ids."""
    import tinygpt_amd as tg
    from test_gpu_sampler import _history_at_top_batch

    g = np.random.default_rng(47 + split)
    V = 12000
    x, params, u, hist, hist_len = _history_at_top_batch(g, 6, V, oracle, H_=256)
    _check(sim, oracle, x, params, u, hist, hist_len, hint=tg.batch_hint(params, V), split=split, kept_cap=64)


def test_k64_bf16_and_mask(sim, oracle):
    import tinygpt_amd as tg
    from tinygpt_amd import workloads as W

    g = np.random.default_rng(45)
    V = 3000
    x, params, u, hist, hist_len = _batch(45, 8, V, oracle)
    params = _k64_params(g, params, V)
    table = g.integers(0, 1 << 32, size=(3, (V + 31) // 32), dtype=np.uint64).astype(np.uint32)
    table[1] &= np.uint32(0x00010001)
    table[2] = 0
    params["mask_state"] = np.array([0, 1, 2, -1, 0, 1, -1, 2])
    _check(sim, oracle, W.f32_to_bf16_bits(x), params, u, hist, hist_len, mask=table,
           hint=tg.batch_hint(params, V), split=3, kept_cap=64)


def _check_conc(sim, oracle, x, params, u, hist, hist_len, mask=None, split=None, repeat=3, xmap=True):
    """The k64 kernel with every workgroup of the launch running at once, so
    that split rows exchange their row-wide bound; `repeat` calls on one
    handle (each call's ids must equal the first's: the exchange state, the
    epoch and the cleared list entries carry over calls)."""
    import tinygpt_amd as tg

    V = x.shape[1]
    env = {} if xmap else {"TGS_XMAP": "0"}
    r = sim.run_sample(x, params, u, hist, hist_len, mask_table=mask, kept_cap=64, hint=tg.batch_hint(params, V),
                       split=split, concurrent=True, repeat=repeat, env_extra=env)
    o = oracle.sample_batch(x, params, u, hist=hist, hist_len=hist_len, mask_table=mask, kept_cap=64,
                            want_post=True)
    assert len(r["launches"]) == repeat  # one k64 launch per call
    return r, o, H.compare(r, o, params, V, what="sim-concurrent")


def _c2_like(g, B, V, oracle, H_=128):
    """C2's statistics at a simulated size: N(0, 3^2), 8 spikes at 12.0 per
    row (ties), Zipf history, presence and frequency penalties, top-k 50."""
    from tinygpt_amd import workloads as W

    x = W.normal_f32(g, (B, V), 3.0)
    for b in range(B):
        x[b, g.choice(V, size=8, replace=False)] = 12.0
    params = oracle.make_params(B, temperature=0.7, top_k=50, top_p=0.9, presence=0.5, frequency=0.3)
    hist = W.zipf_ids(g, 0, V, shape=(B, H_))
    hist_len = np.full(B, H_, np.int32)
    u = W.uniforms(g, B)
    return x, params, u, hist, hist_len


@pytest.mark.parametrize("split,xmap", [(2, True), (8, False)])
def test_k64_exchange_c2_like(sim, oracle, split, xmap):
    """Split rows sharing the row-wide bound (C2's statistics), with and
    without the XCD-aware workgroup order, over three calls."""
    g = np.random.default_rng(60 + split)
    x, params, u, hist, hist_len = _c2_like(g, 8 if xmap else 2, 40000, oracle)
    params["temperature"][1] = 0.0  # a greedy row
    params["top_k"][0] = 1
    _check_conc(sim, oracle, x, params, u, hist, hist_len, split=split, xmap=xmap)


def test_k64_exchange_mixed_rows(sim, oracle):
    """The exchange on the random batches' rows (ties, special values, equal
    rows, ascending rows whose top ids share one chunk, penalties that lift
    or sink history ids), k up to 64: rows whose candidates outgrow a list
    or the staging take the sorted top-k and exact paths."""
    g = np.random.default_rng(63)
    V = 20000
    x, params, u, hist, hist_len = _batch(63, 7, V, oracle)
    params = _k64_params(g, params, V)
    _check_conc(sim, oracle, x, params, u, hist, hist_len, split=2, xmap=False)


def test_k64_exchange_mask_bf16(sim, oracle):
    """The exchange with a grammar mask (dense, sparse and empty rows) on
    bf16 logits."""
    from tinygpt_amd import workloads as W

    g = np.random.default_rng(64)
    V = 24000
    x, params, u, hist, hist_len = _c2_like(g, 4, V, oracle, H_=64)
    params = _k64_params(g, params, V)
    table = g.integers(0, 1 << 32, size=(3, (V + 31) // 32), dtype=np.uint64).astype(np.uint32)
    table[1] &= np.uint32(0x00100001)
    table[2] = 0
    params["mask_state"] = np.array([0, 1, 2, -1])
    _check_conc(sim, oracle, W.f32_to_bf16_bits(x), params, u, hist, hist_len, mask=table, split=3, xmap=False)


def test_k64_merge_give_up_leaves_nothing_behind(sim, oracle):
    """Merges whose wait gives up: three leading calls on other inputs (every
    row reversed) with the merge's poll limit forced to 0 from the host,
    every workgroup of the launch running at once, so that merging
    workgroups give up (id -4) before some lists are out, and those lists
    are published after the merge is over.  The two calls after them, on
    the real inputs and the default limit, take none of the entries left
    behind: their ids equal the oracle's (and each other's).  On the
    allocation-free entry point's static workspace, which keeps its lists
    for the life of the process.  (How many merges give up depends on the
    threads' schedule; the count is printed.)"""
    import re

    import tinygpt_amd as tg

    g = np.random.default_rng(66)
    B, V = 4, 24000
    x, params, u, hist, hist_len = _c2_like(g, B, V, oracle, H_=64)
    r = sim.run_sample(x, params, u, hist, hist_len, kept_cap=64, hint=tg.batch_hint(params, V), split=4,
                       concurrent=True, repeat=2, noalloc=True,
                       env_extra={"TGS_SIM_FIRST_MERGE_SPINS": "0", "TGS_XMAP": "0"})
    m = re.search(r"leading calls: (\d+) rows gave up", r["stdout"])
    assert m, r["stdout"]
    print(f"leading calls: {m.group(1)} of {3 * B} rows gave up")
    o = oracle.sample_batch(x, params, u, hist=hist, hist_len=hist_len, kept_cap=64, want_post=True)
    k64 = [l for l in r["launches"] if l == (B * 4, 512)]
    assert len(k64) == 5  # three leading calls and two more (the static workspace adds its set-up fill once)
    H.compare(r, o, params, V, what="sim-after-give-up")


def test_k64_exchange_history_at_top(sim, oracle):
    """The exchange where the rows' largest logits are penalised history ids."""
    from test_gpu_sampler import _history_at_top_batch

    g = np.random.default_rng(65)
    x, params, u, hist, hist_len = _history_at_top_batch(g, 4, 16000, oracle, H_=256)
    _check_conc(sim, oracle, x, params, u, hist, hist_len, split=4, xmap=False)


@pytest.mark.parametrize("bf16", [False, True])
def test_token_logprobs(sim, oracle, bf16):
    """tgs_token_logprobs: one workgroup per row, rows split into chunks
    (few rows of 20000 ids), an odd stride (unaligned rows, scalar path) and
    special values, within 1e-4 + 1e-6 |x| of the float64 oracle."""
    from tinygpt_amd import workloads as W

    g = np.random.default_rng(70)
    for B, V, stride in ((5, 3000, 3000), (3, 20000, 20000), (4, 999, 1001)):
        x = g.normal(0.0, 3.0, (B, stride)).astype(np.float32)
        x[0, 5] = -np.inf
        if B > 3:
            x[3, :] = -np.inf
            x[2, 9] = np.nan
        if bf16:
            if stride % 8:
                continue
            x = W.f32_to_bf16_bits(x)
        tok = g.integers(0, V, B)
        tok[-1] = V  # outside: NaN
        lp, lse = sim.run_logprob(x, tok, V=V)
        r_lp, r_lse = oracle.token_logprobs(x, tok, V=V)
        for got, ref in ((lp, r_lp), (lse, r_lse)):
            nan = np.isnan(ref)
            np.testing.assert_array_equal(np.isnan(got), nan)
            assert np.all(np.abs(got[~nan] - ref[~nan]) <= 1e-4 + 1e-6 * np.abs(ref[~nan]))


def test_mask_rows_from_dfa(sim, oracle):
    """tgs_mask_rows_from_dfa under ASan: tool-tag rows for several states,
    a complete state with an EOS id, rows outside the table skipped, a token
    longer than the bytes read up front; the class table in LDS, the full
    table in global memory, and a byte mapped to a class outside the table;
    read back through greedy rows."""
    from tinygpt_amd import grammar as G

    g = np.random.default_rng(80)
    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    pieces = [b"[", b"]", b"POINT", b":", b"none", b",", b"TYPE", b"up", b" ", b"-", b"\xc3\xa9", b"12", b"x"]
    toks = [b""] + [b"".join(g.choice(pieces) for _ in range(g.integers(1, 4))) for _ in range(600)]
    toks.append(bytes(range(65, 65 + 30)))
    V = len(toks)
    off, data = G.token_csr(toks)
    # more states than one workgroup walks together, the last group partial
    hist = [b"", b"ok [", b"ok [POINT:1", b"[TYPE:ab", b"[POINT:none]", b"[SCROLL:", b"[KEY:a", b"ok",
            b"[POINT:1,2:x", b"[OPEN_APP:S"]
    nh = len(hist)
    states = np.array([d.walk(0, h) for h in hist] + [0, 0], np.int32)
    rows = np.array(list(range(nh)) + [-1, 99], np.int32)
    bc, ct = d.byte_classes()
    bad = bc.copy()
    bad[ord("x")] = ct.shape[1]  # a class outside the table rejects the byte
    t_bad = d.trans.copy()
    t_bad[:, ord("x")] = -1
    cases = [(bc, ct, d.trans),  # 40 classes: the table in LDS
             (np.arange(256, dtype=np.uint8), d.trans, d.trans),  # 256 columns: the table in global memory
             (bad, ct, t_bad)]
    for byte_class, trans, full in cases:
        post = sim.run_maskbuild(byte_class, trans, d.complete.astype(np.uint8), off, data, states, rows,
                                 n_rows=nh + 1, eos=3)
        want = oracle.dfa_mask_rows(full, d.complete, toks, states[:nh], eos=3)
        for i in range(nh):
            allowed = np.array([(int(want[i, v >> 5]) >> (v & 31)) & 1 for v in range(V)], dtype=bool)
            np.testing.assert_array_equal(post[i] == 0.0, allowed)
        assert (post[nh] == 0.0).all()  # untouched row
    # more states than one workgroup takes (a second workgroup row)
    st70 = np.resize(states[:nh], 70).astype(np.int32)
    post = sim.run_maskbuild(bc, ct, d.complete.astype(np.uint8), off, data, st70, np.arange(70, dtype=np.int32),
                             n_rows=70, eos=3)
    want = oracle.dfa_mask_rows(d.trans, d.complete, toks, st70, eos=3)
    for i in (0, 63, 64, 69):
        allowed = np.array([(int(want[i, v >> 5]) >> (v & 31)) & 1 for v in range(V)], dtype=bool)
        np.testing.assert_array_equal(post[i] == 0.0, allowed)



def test_mask_rows_offsets_outside_the_bytes(sim, oracle):
    """Token offsets that do not give a range inside the byte buffer (a
    negative start, a range that ends before it starts, an end past the
    buffer, the last token running past it) read as empty tokens, never
    allowed, under ASan with a byte buffer of exactly its length: no read
    leaves it.  Every other token keeps the bytes its offsets give, and the
    rows match the DFA replay oracle over those tokens, in both the LDS and
    the global kernel."""
    from tinygpt_amd import grammar as G

    g = np.random.default_rng(82)
    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    pieces = [b"[", b"]", b"POINT", b":", b"none", b",", b"TYPE", b"up", b" ", b"12", b"x"]
    toks = [b"".join(g.choice(pieces) for _ in range(g.integers(1, 4))) for _ in range(300)]
    toks.append(b"[" + b"POINT:" * 4)  # longer than the bytes read up front
    off, data = G.token_csr(toks)
    off = off.astype(np.int64)
    n = len(data)
    off[10] = -5               # token 9 ends below 0, token 10 starts below 0
    off[20] = off[19] - 1      # token 19 ends before it starts
    off[30] = n + 1000         # token 29 ends past the buffer, token 30 starts past it
    off[40] = off[42]          # token 39 longer, token 40 empty, token 41 intact
    off[-1] = n + 7            # the last token runs past the buffer
    off = off.astype(np.int32)
    V = len(toks)
    got_toks = []
    for v in range(V):
        s, e = int(off[v]), int(off[v + 1])
        got_toks.append(bytes(data[s:e]) if 0 <= s < e <= n else b"")
    for v in (9, 10, 19, 29, 30, 40, V - 1):
        assert got_toks[v] == b""
    hist = [b"", b"ok [", b"[POINT:1", b"[TYPE:ab", b"[POINT:none]"]
    states = np.array([d.walk(0, h) for h in hist], np.int32)
    rows = np.arange(len(hist), dtype=np.int32)
    bc, ct = d.byte_classes()
    want = oracle.dfa_mask_rows(d.trans, d.complete, got_toks, states, eos=3)
    for byte_class, trans in ((bc, ct), (np.arange(256, dtype=np.uint8), d.trans)):
        post = sim.run_maskbuild(byte_class, trans, d.complete.astype(np.uint8), off, data, states, rows,
                                 n_rows=len(hist), eos=3)
        for i in range(len(hist)):
            allowed = np.array([(int(want[i, v >> 5]) >> (v & 31)) & 1 for v in range(V)], dtype=bool)
            np.testing.assert_array_equal(post[i] == 0.0, allowed)
            assert not allowed[[9, 10, 19, 29, 30, 40, V - 1]].any()


def test_mask_rows_many_tool_tag_states(sim, oracle):
    """80 states of the tool-tag DFA (five workgroup rows of the LDS kernel,
    MASK_SPW_LDS = 16 states each, two of the global kernel, MASK_SPW = 64)
    through the class table in LDS and the 256-column table in global
    memory (the GPU test takes all 434)."""
    from tinygpt_amd import grammar as G

    g = np.random.default_rng(81)
    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    pieces = [b"[", b"]", b"POINT", b":", b"none", b",", b"CLICK", b"TYPE", b"up", b" ", b"-", b"12", b"x", b"A"]
    toks = [b""] + [b"".join(g.choice(pieces) for _ in range(g.integers(1, 4))) for _ in range(40)]
    V = len(toks)
    off, data = G.token_csr(toks)
    states = np.arange(80, dtype=np.int32)
    want = oracle.dfa_mask_rows(d.trans, d.complete, toks, states, eos=5)
    bits = np.unpackbits(want.view(np.uint8), axis=1, bitorder="little")[:, :V].astype(bool)
    bc, ct = d.byte_classes()
    for byte_class, trans in ((bc, ct), (np.arange(256, dtype=np.uint8), d.trans)):
        post = sim.run_maskbuild(byte_class, trans, d.complete.astype(np.uint8), off, data, states, states,
                                 n_rows=len(states), eos=5)
        np.testing.assert_array_equal(post == 0.0, bits)

def _spec_case(seed, B, k, V, T, bf16=False):
    from tinygpt_amd import workloads as W

    c = W.config5(B=B, k=k, V=V, seed_offset=seed, T=1.0)
    c["T"][:] = T
    c["dtok"][::3, 0] = np.argmin(c["target"][::3, 0], axis=-1)  # early rejections
    if B > 2:
        c["T"][2] = 0.0  # a greedy sequence among stochastic ones
    if bf16:
        c["target"] = W.f32_to_bf16_bits(c["target"])
        c["draft"] = W.f32_to_bf16_bits(c["draft"])
    return c


def _spec_check(sim, oracle, c):
    n_s, out_s = sim.run_spec(c["target"], c["draft"], c["dtok"], c["T"], c["u_acc"], c["u_res"])
    o = oracle.spec_verify_batch(c["target"], c["draft"], c["dtok"], c["T"], c["u_acc"], c["u_res"])
    np.testing.assert_array_equal(n_s, o["n_acc"])
    np.testing.assert_array_equal(out_s, o["out"])
    return o


@pytest.mark.parametrize("T", [1.0, 0.5])
def test_spec_blocks_decide_mass_draw(sim, oracle, T):
    # V = 2500: three blocks of 1024 ids, the last one partial, rows not
    # 16-byte aligned (scalar edge loads)
    o = _spec_check(sim, oracle, _spec_case(11, 6, 3, 2500, T))
    assert (o["n_acc"] >= 0).all()


def test_spec_bf16_aligned(sim, oracle):
    _spec_check(sim, oracle, _spec_case(12, 4, 2, 2048, 1.0, bf16=True))


def test_spec_zero_residual_falls_back_to_target(sim, oracle):
    # draft == target and the first draft token has probability 0 in both:
    # rejected (ratio 0), residual 0 everywhere -> draw from the target row
    from tinygpt_amd import workloads as W

    c = W.config5(B=3, k=2, V=1500, seed_offset=13)
    c["draft"] = c["target"][:, :2].copy()
    c["target"][np.arange(3), 0, c["dtok"][:, 0]] = -np.inf
    c["draft"][np.arange(3), 0, c["dtok"][:, 0]] = -np.inf
    o = _spec_check(sim, oracle, c)
    assert (o["n_acc"] == 0).all() and (o["info"]["resampled"] == 2).all()


@pytest.mark.parametrize("T", [1.0, 0.5, 0.7])
def test_spec_special_blocks(sim, oracle, T):
    """The GPU test's batch of -inf, NaN and +inf blocks between finite ones
    (deferred block masses across blocks stored at once), greedy and NaN-T
    sequences among them."""
    from test_gpu_spec import special_blocks_case

    _spec_check(sim, oracle, special_blocks_case(T))


def test_spec_invalid_rows(sim, oracle):
    from tinygpt_amd import workloads as W

    c = W.config5(B=4, k=2, V=64, seed_offset=4)
    c["dtok"][0, 1] = 64
    c["T"][1] = np.nan
    c["u_acc"][2, 0] = 1.0
    _spec_check(sim, oracle, c)


@pytest.mark.parametrize("mode,n", [("div", 20_000_000), ("exp", 20_000_000), ("q40", 10_000_000),
                                    ("divt", 40_000_000),
                                    ("q40exp", 20_000_000), ("pow2fma", 20_000_000)])
def test_device_shortcuts_equal_canonical_ops(sim, mode, n):
    """tg_div_t == IEEE z / T (the temperature divide, every mode, with zeros,
    infinities, NaN, denormals and huge logits among the inputs),
    tg_div_rcp == IEEE a / b (weights over softmax denominators),
    tg_expf_nonpos == tg_expf on x <= 0 / -inf / NaN, f64-summed
    tg_q40d == tg_q40, the one-step mass tg_q40d_exp_nonpos == tg_q40d of
    tg_expf_nonpos, and a power-of-two temperature's fused fma(z, rT, -m)
    giving the same mass as z rT - m, on the device header compiled for the
    host."""
    import subprocess

    r = subprocess.run([os.path.join(HERE, "cpu_sim", "build", "numerics"), mode, str(n), "12345"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 mismatches" in r.stdout


def _topp_batch(seed, B, V, oracle, bf16=False):
    x, params, u, hist, hist_len = _batch(seed, B, V, oracle)
    g = np.random.default_rng(seed)
    params["top_k"] = g.choice([0, -1, V, V + 7], size=B)  # no top-k: the top-p kernel
    params["top_p"][::2] = 0.9
    if bf16:
        from tinygpt_amd import workloads as W

        x = W.f32_to_bf16_bits(x)
    return x, params, u, hist, hist_len


def test_topp_kernel_rows(sim, oracle):
    x, params, u, hist, hist_len = _topp_batch(21, 10, 3000, oracle)
    r, _, _ = _check(sim, oracle, x, params, u, hist, hist_len)
    assert (10, 1024) in r["launches"]  # the top-p kernel ran


def test_topp_kernel_mask_bf16(sim, oracle):
    x, params, u, hist, hist_len = _topp_batch(22, 6, 2100, oracle, bf16=True)
    g = np.random.default_rng(5)
    words = (2100 + 31) // 32
    mask = g.integers(0, 1 << 32, size=(4, words), dtype=np.uint64).astype(np.uint32)
    mask[1] = 0
    params["mask_state"] = g.integers(-1, 4, size=6)
    _check(sim, oracle, x, params, u, hist, hist_len, mask=mask)


def test_topp_kernel_bucket_overflow(sim, oracle):
    # flat rows: every id in the first bucket (more than the ranked capacity)
    B, V = 3, 5000
    x = np.full((B, V), 0.75, np.float32)
    x[1, ::3] = 0.7
    params = oracle.make_params(B, temperature=1.0, top_k=0, top_p=0.37)
    params["top_p"][2] = 1.0
    u = np.array([0.1, 0.5, 0.99], np.float32)
    _check(sim, oracle, x, params, u, None, None)


def test_topp_kernel_dense_rows_in_registers(sim, oracle):
    """Register-resident rows whose allowed ids outnumber the LDS packing
    capacity: the later passes run over the registers (one row masked down
    to a packable count for contrast)."""
    import tinygpt_amd as tg

    B, V = 3, 24576
    g = np.random.default_rng(62)
    x = g.normal(0.0, 2.0, (B, V)).astype(np.float32)
    mask = np.full((1, V // 32), 0x0F0F0F0F, np.uint32)
    params = oracle.make_params(B, temperature=[1.0, 0.8, 1.2], top_k=0, top_p=[0.9, 0.5, 1.0],
                                mask_state=[-1, -1, 0])
    u = g.random(B).astype(np.float32)
    hint = tg.batch_hint(params, V)
    r, _, _ = _check(sim, oracle, x, params, u, None, None, mask=mask, hint=hint, kept_cap=64)
    assert r["launches"] == [(B, 1024)]


@pytest.mark.parametrize("bf16", [False, True])
def test_topp_kernel_serves_whole_batch(sim, oracle, bf16):
    """Every sampling row without a usable top-k (the hint's min_top_k == V):
    one top-p launch serves the greedy rows too.  Masked rows, an all-masked
    row, an invalid row, quantized logits (buckets past one wave) and top-p
    off are mixed in."""
    import tinygpt_amd as tg

    B, V = 9, 2048
    g = np.random.default_rng(61)
    x = g.normal(0.0, 2.5, (B, V)).astype(np.float32)
    x[3] = np.round(x[3] * 2.0) / 2.0
    x[4] = np.round(x[4])
    words = V // 32
    mask = g.integers(0, 1 << 32, size=(3, words), dtype=np.uint64).astype(np.uint32)
    mask[1] = 0
    params = oracle.make_params(B, temperature=1.0, top_k=0, top_p=0.95,
                                mask_state=[0, -1, 2, -1, -1, 1, 0, -1, 2])
    params["temperature"][[0, 2, 6]] = 0.0  # greedy
    params["temperature"][7] = np.nan  # invalid: -2
    params["top_p"][4] = 1.0
    params["top_k"][8] = V + 5
    u = g.random(B).astype(np.float32)
    if bf16:
        from tinygpt_amd import workloads as W

        x = W.f32_to_bf16_bits(x)
    hint = tg.batch_hint(params, V)
    assert hint == V and hint.min_top_k == V
    r, _, _ = _check(sim, oracle, x, params, u, None, None, mask=mask, hint=hint)
    assert r["launches"] == [(B, 1024)]  # the top-p kernel alone
    # a row with a usable top-k breaks the hint's promise: -3
    params["top_k"][1] = 5
    r = sim.run_sample(x, params, u, mask_table=mask, hint=hint, post=False)
    o = oracle.sample_batch(x, params, u, mask_table=mask)
    expect = o["ids"].copy()
    expect[1] = -3
    np.testing.assert_array_equal(r["ids"], expect)


def _topk_batch(seed, B, V, oracle, bf16=False):
    x, params, u, hist, hist_len = _batch(seed, B, V, oracle)
    g = np.random.default_rng(seed)
    params["top_k"] = g.choice([1, 3, 64, 65, 200, 1000, 1024], size=B)
    if bf16:
        from tinygpt_amd import workloads as W

        x = W.f32_to_bf16_bits(x)
    return x, params, u, hist, hist_len


def test_topk_kernel_rows(sim, oracle):
    import tinygpt_amd as tg

    # hint above 64: the register-resident top-k kernel (V * 4 bytes is a whole number of vectors)
    x, params, u, hist, hist_len = _topk_batch(31, 9, 3000, oracle)
    r, _, _ = _check(sim, oracle, x, params, u, hist, hist_len, hint=tg.batch_hint(params, 3000))
    assert r["launches"] == [(9, 1024)]  # one 1024-thread workgroup per row


def test_topk_kernel_bf16_mask(sim, oracle):
    import tinygpt_amd as tg

    x, params, u, hist, hist_len = _topk_batch(32, 6, 2048, oracle, bf16=True)
    g = np.random.default_rng(6)
    mask = g.integers(0, 1 << 32, size=(3, 64), dtype=np.uint64).astype(np.uint32)
    mask[2] = 0
    params["mask_state"] = g.integers(-1, 3, size=6)
    r, _, _ = _check(sim, oracle, x, params, u, hist, hist_len, mask=mask, hint=tg.batch_hint(params, 2048))
    assert r["launches"] == [(6, 1024)]


@pytest.mark.parametrize("bf16", [False, True])
def test_topk_kernel_tail_buckets(sim, oracle, bf16):
    """Rows that drive every path of the top-k kernel's bucket tail: ties
    filling a bucket past one wave (counting ranks) and past the ranking
    capacity (radix selections within the bucket), kept ids in the mass-0
    bucket (y - m <= -32) with top-p off (cut = k-th id), a top-p target of
    0, greedy rows, rows of mostly or only negative logits."""
    import tinygpt_amd as tg

    B, V = 7, 3000
    g = np.random.default_rng(41)
    x = np.empty((B, V), np.float32)
    x[0] = np.round(g.normal(0.0, 2.0, V) * 4.0) / 4.0  # ~30 distinct values: ties
    x[1] = 0.25
    x[1, [7, 900, 2999]] = [2.0, 1.0, 1.5]  # one huge bucket
    x[2] = g.normal(0.0, 1.0, V)  # T = 0.01: most kept ids carry mass 0
    x[3] = g.normal(0.0, 3.0, V) - 6.0
    x[4] = np.round(g.normal(0.0, 1.0, V) * 2.0) / 2.0
    x[5] = g.normal(0.0, 2.0, V) - 50.0  # all negative: the bound from group minima
    x[6] = np.round(g.normal(0.0, 2.0, V))
    params = oracle.make_params(B, temperature=[1.0, 0.7, 0.01, 1.3, 0.5, 0.0, 2.0],
                                top_k=[1000, 1024, 500, 800, 1024, 5, 64], top_p=[0.9, 0.5, 1.0, 1e-9, 1.0, 1.0, 0.999])
    u = g.random(B).astype(np.float32)
    if bf16:
        from tinygpt_amd import workloads as W

        x = W.f32_to_bf16_bits(x)
    r, _, _ = _check(sim, oracle, x, params, u, None, None, hint=tg.batch_hint(params, V))
    assert r["launches"] == [(B, 1024)]


def test_topk_kernel_candidate_overflow(sim, oracle):
    import tinygpt_amd as tg

    # one value everywhere but a few ids: every id ties at the bound, more
    # candidates than the list holds
    B, V = 2, 6000
    x = np.full((B, V), 0.5, np.float32)
    x[0, [5, 77, 4000]] = 3.0
    params = oracle.make_params(B, temperature=0.9, top_k=700, top_p=0.8)
    u = np.array([0.3, 0.95], np.float32)
    r, _, _ = _check(sim, oracle, x, params, u, None, None, hint=tg.batch_hint(params, V))
    assert r["launches"] == [(2, 1024)]
